"""GPU parity of the paged KV cache ops and decode attention against
oracle/attention.py, through the C ABI (LayerBlocksHolder, PagedAttention).

Bars: cache writes and restores bit-exact (pure data movement); attention
output within max|o - o_ref| <= 1e-2 * ||o_ref row||_inf of the float64
oracle (softmax and both products in fp32 on the GPU, one fp16 rounding).
Covers block sizes 16/32, head sizes 64/128/256, grouped-query heads (up to
8 per kv head), ALiBi, ragged contexts (1 token, block edges, partitioned
long contexts), padding slots, scattered and separately allocated blocks,
determinism and the error statuses.  Every case prints its name before
touching the GPU.
"""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest
import torch

from hip_extends import _lib
from operators import flags
from operators.core.attention.common import AttentionConfig
from operators.core.attention.real_page import PagedAttention
from operators.core.block.common import BlockInfo
from operators.core.block.real import LayerBlocksHolder
from oracle import attention as A
from oracle import gptq

pytestmark = pytest.mark.gpu
TOL = 1e-2


def say(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture
def block_size(request):
    old = flags.BLOCK_SIZE
    flags.BLOCK_SIZE = request.param
    yield request.param
    flags.BLOCK_SIZE = old


def _fill(holder, ctxs, kvh, hs, bs, seed, dev):
    """Write each sequence's k, v through reshape_and_cache into scattered
    blocks; returns tables, the token-major k, v and the numpy caches."""
    rng = np.random.default_rng(seed)
    nblocks = holder.layer_key_ptr_table_cpu.numel()
    per = [(c + bs - 1) // bs for c in ctxs]
    perm = rng.permutation(nblocks)
    tables = np.zeros((len(ctxs), max(per)), np.int32)
    kc, vc = A.empty_cache(nblocks, kvh, hs, bs, fill=0.0)
    nxt = 0
    for s, c in enumerate(ctxs):
        tables[s, :per[s]] = perm[nxt:nxt + per[s]]
        nxt += per[s]
        k = rng.standard_normal((c, kvh, hs)).astype(np.float16)
        v = rng.standard_normal((c, kvh, hs)).astype(np.float16)
        slots = np.array([tables[s, t // bs] * bs + t % bs for t in range(c)], np.int64)
        holder.kv_tensor_to_slots_with_convert(torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev),
                                               torch.from_numpy(slots).to(dev))
        A.reshape_and_cache(k, v, kc, vc, slots)
    return tables, kc, vc


@pytest.mark.parametrize("block_size", [16, 32], indirect=True)
def test_cache_ops_bit_exact(hip_device, block_size):
    bs = block_size
    info = BlockInfo(head_dim=128, num_key_value_heads=4)
    holder = LayerBlocksHolder.create_contigious_cacher(info, 12, hip_device)
    kt, vt = holder.contigious_kv_tenosr
    kt.zero_()
    vt.zero_()
    rng = np.random.default_rng(bs)
    key = rng.standard_normal((30, 4, 128)).astype(np.float16)
    val = rng.standard_normal((30, 4, 128)).astype(np.float16)
    slots = rng.permutation(12 * bs)[:30].astype(np.int64)
    slots[[2, 11]] = -1
    say(f"reshape_and_cache bs={bs}")
    holder.kv_tensor_to_slots_with_convert(torch.from_numpy(key).to(hip_device),
                                           torch.from_numpy(val).to(hip_device),
                                           torch.from_numpy(slots).to(hip_device))
    torch.cuda.synchronize()
    kc, vc = A.empty_cache(12, 4, 128, bs, fill=0.0)
    A.reshape_and_cache(key, val, kc, vc, slots)
    assert np.array_equal(kt.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(vt.cpu().numpy().view(np.uint16), vc.view(np.uint16))
    say(f"restore_from_cache bs={bs}")
    k2, v2 = holder.kv_tensor_from_slots_with_convert_with_create(torch.from_numpy(slots).to(hip_device))
    torch.cuda.synchronize()
    keep = slots >= 0
    assert np.array_equal(k2.cpu().numpy()[keep].view(np.uint16), key[keep].view(np.uint16))
    assert np.array_equal(v2.cpu().numpy()[keep].view(np.uint16), val[keep].view(np.uint16))


CASES = [
    # seqs' context lengths, heads, kv heads, head size, block size, alibi
    ([1, 7, 32, 20], 8, 8, 128, 32, False),      # one block: single partition
    ([1, 16, 17, 100], 8, 8, 128, 16, False),
    ([5, 64, 200], 8, 2, 64, 32, False),         # 4 query heads per kv head
    ([512] * 8, 32, 32, 128, 16, False),         # the 7B stage's shape
    ([300, 41], 32, 4, 128, 16, True),           # 8 per kv head, ALiBi
    ([1500, 2049, 3], 4, 4, 128, 32, False),     # partitions of 512 tokens
    ([33, 90], 6, 3, 256, 16, False),
    # head sizes that are not multiples of 64: some lanes hold no last key
    # slice or value dim
    ([1, 37, 600], 8, 8, 80, 16, False),
    ([70, 513], 8, 2, 80, 32, True),
    ([1, 129, 40], 12, 12, 96, 16, False),
    ([260, 17], 16, 2, 96, 32, False),
    ([3, 100, 1100], 8, 1, 112, 16, False),
    ([45, 64], 4, 4, 112, 32, True),
    # more than half as many (sequence, kv head) pairs as CUs, contexts up to
    # 1024 tokens, 16-token blocks: one 16-wave workgroup per pair over the
    # whole context (no combine launch) on a 256-CU device
    ([1000, 3, 517, 64, 250, 1, 33, 768], 24, 24, 80, 16, False),
    ([200, 1024, 7, 45, 96, 300, 12, 640], 96, 24, 96, 16, True),
    ([129, 1, 800, 300], 384, 48, 64, 16, False),
    ([5, 900, 333, 64, 1, 2], 128, 32, 112, 16, False),
    ([1, 17, 1024, 511, 512, 33, 300, 64, 100], 64, 16, 128, 16, False),
    # the 16-wave form past 32 blocks, where a wave's third (and fourth)
    # block reloads a register slot after the first blocks' q . k and p . v:
    # the 7B stage's shape as its contexts grow past 512 (ALiBi added), and
    # 4 query heads per kv head at head size 64
    ([640, 513, 600, 576, 1, 530, 700, 520], 32, 32, 128, 16, True),
    ([1000, 520, 3, 777], 160, 40, 64, 16, False),
]


@pytest.mark.parametrize("ctxs,heads,kvh,hs,bs,alibi", CASES)
def test_paged_attention(hip_device, ctxs, heads, kvh, hs, bs, alibi):
    old = flags.BLOCK_SIZE
    flags.BLOCK_SIZE = bs
    try:
        info = BlockInfo(head_dim=hs, num_key_value_heads=kvh)
        nblocks = sum((c + bs - 1) // bs for c in ctxs) + 5
        holder = LayerBlocksHolder.create_contigious_cacher(info, nblocks, hip_device)
        say(f"paged attention ctxs={ctxs} heads={heads}/{kvh} hs={hs} bs={bs} alibi={alibi}")
        tables, kc, vc = _fill(holder, ctxs, kvh, hs, bs, len(ctxs) * heads + hs, hip_device)
        rng = np.random.default_rng(99)
        q = rng.standard_normal((len(ctxs), heads, hs)).astype(np.float16)
        slopes = (2.0 ** -np.arange(1, heads + 1) * 8 / heads).astype(np.float32) if alibi else None
        att = PagedAttention(AttentionConfig(heads * hs, hs, heads, kvh, heads // kvh))
        lens = torch.tensor(ctxs, dtype=torch.int32, device=hip_device)
        out = att.forward(torch.from_numpy(q).to(hip_device), max(ctxs), lens,
                          torch.from_numpy(tables).to(hip_device), holder,
                          None if slopes is None else torch.from_numpy(slopes).to(hip_device))
        again = att.forward(torch.from_numpy(q).to(hip_device), max(ctxs), lens,
                            torch.from_numpy(tables).to(hip_device), holder,
                            None if slopes is None else torch.from_numpy(slopes).to(hip_device))
        torch.cuda.synchronize()
        assert torch.equal(out, again)  # deterministic
        ref = A.paged_attention(q, kc, vc, tables, np.array(ctxs), att.scale, slopes)
        y = out.float().cpu().numpy()
        assert np.all(np.isfinite(y))
        ok, worst = gptq.within_tolerance(y.reshape(-1, hs), ref.reshape(-1, hs), TOL)
        assert ok, f"worst error ratio {worst:.3f}"
    finally:
        flags.BLOCK_SIZE = old


def test_separately_allocated_blocks(hip_device):
    """A pointer table over blocks allocated one by one (no contiguous backing),
    the reference's swap-in case."""
    bs, kvh, hs = flags.BLOCK_SIZE, 4, 128
    info = BlockInfo(head_dim=hs, num_key_value_heads=kvh)
    ks = [torch.zeros(info.key_block_shape, dtype=torch.float16, device=hip_device) for _ in range(9)]
    vs = [torch.zeros(info.value_block_shape, dtype=torch.float16, device=hip_device) for _ in range(9)]
    kp = [t.data_ptr() for t in ks]
    vp = [t.data_ptr() for t in vs]
    kc_t, vc_t = torch.tensor(kp), torch.tensor(vp)
    holder = LayerBlocksHolder(info, kc_t.to(hip_device), vc_t.to(hip_device), kc_t, vc_t, kp, vp)
    assert not holder.is_contigious
    ctxs = [100, 65]
    say("paged attention over separately allocated blocks")
    tables, kc, vc = _fill(holder, ctxs, kvh, hs, bs, 5, hip_device)
    q = np.random.default_rng(6).standard_normal((2, 8, hs)).astype(np.float16)
    att = PagedAttention(AttentionConfig(8 * hs, hs, 8, kvh, 2))
    out = att.forward(torch.from_numpy(q).to(hip_device), max(ctxs),
                      torch.tensor(ctxs, dtype=torch.int32, device=hip_device),
                      torch.from_numpy(tables).to(hip_device), holder)
    torch.cuda.synchronize()
    ref = A.paged_attention(q, kc, vc, tables, np.array(ctxs), att.scale)
    ok, worst = gptq.within_tolerance(out.float().cpu().numpy().reshape(-1, hs), ref.reshape(-1, hs), TOL)
    assert ok, worst


def test_attention_statuses(hip_device):
    lib = _lib.load()
    sz = ctypes.c_size_t(0)
    say("paged attention statuses")
    assert lib.dw4_paged_attention_workspace_size(2, 8, 8, 72, 16, 100, ctypes.byref(sz)) == \
        _lib.DW4_ERR_UNSUPPORTED  # head size not served
    for hs in (64, 80, 96, 112, 128, 256):
        assert lib.dw4_paged_attention_workspace_size(2, 8, 8, hs, 16, 100,
                                                      ctypes.byref(sz)) == _lib.DW4_OK
    if torch.cuda.get_device_properties(hip_device).multi_processor_count == 256:
        # the stage shape (8 x 32 (sequence, kv head) pairs, 512 tokens): one
        # 16-wave workgroup per pair, no partitions, no workspace; a small
        # batch keeps the partitioned form
        assert lib.dw4_paged_attention_workspace_size(8, 32, 32, 128, 16, 512,
                                                      ctypes.byref(sz)) == _lib.DW4_OK
        assert sz.value == 0
        assert lib.dw4_paged_attention_workspace_size(2, 8, 8, 128, 16, 512,
                                                      ctypes.byref(sz)) == _lib.DW4_OK
        assert sz.value > 0
    assert lib.dw4_paged_attention_workspace_size(2, 36, 4, 128, 16, 100, ctypes.byref(sz)) == \
        _lib.DW4_ERR_UNSUPPORTED  # 9 query heads per kv head
    assert lib.dw4_paged_attention_workspace_size(2, 8, 8, 128, 8, 100, ctypes.byref(sz)) == \
        _lib.DW4_ERR_UNSUPPORTED  # block size 8
    q = torch.zeros(4, 8, 128, dtype=torch.float16, device=hip_device)
    o = torch.empty_like(q)
    ptrs = torch.zeros(4, dtype=torch.int64, device=hip_device)
    tab = torch.zeros(4, 64, dtype=torch.int32, device=hip_device)
    lens = torch.ones(4, dtype=torch.int32, device=hip_device)
    need = _lib.paged_attention_workspace_size(4, 8, 8, 128, 16, 1000)
    assert need > 0
    assert lib.dw4_paged_attention(4, 8, 8, 128, 16, q.data_ptr(), 1024, o.data_ptr(), 1024,
                                   ptrs.data_ptr(), ptrs.data_ptr(), 2048, 0.1, tab.data_ptr(),
                                   64, lens.data_ptr(), 1000, None, None, 0, None) == \
        _lib.DW4_ERR_WORKSPACE
    assert lib.dw4_paged_attention(4, 8, 8, 128, 16, q.data_ptr(), 1024, o.data_ptr(), 1024,
                                   ptrs.data_ptr(), ptrs.data_ptr(), 2048, 0.1, tab.data_ptr(),
                                   8, lens.data_ptr(), 1000, None, None, 0, None) == \
        _lib.DW4_ERR_INVALID_ARG  # block table shorter than the context
    assert lib.dw4_reshape_and_cache(3, 4, 100, 16, q.data_ptr(), 400, q.data_ptr(), 400,
                                     ptrs.data_ptr(), ptrs.data_ptr(), 1600, ptrs.data_ptr(),
                                     None) == _lib.DW4_ERR_UNSUPPORTED  # head size % 8


@pytest.mark.parametrize("table_dims", [2, 4], ids=["P_hd", "1_1_P_hd"])
@pytest.mark.parametrize("past", [3, -1])
def test_rope_bit_exact(hip_device, past, table_dims):
    """Tables as [P, hd] and as the rotary modules' [1, 1, P, hd]
    (operators/core/rope/real.py:114,140 in the reference)."""
    from hip_extends.w4a16 import attention_forward_rope_stage_v2_py
    rng = np.random.default_rng(21)
    batch, q_len, heads, kvh, hd = 3, 2, 4, 2, 128
    sin, cos = A.rope_tables(40, hd)
    q = (rng.standard_normal((batch, q_len * heads, hd)) * 3).astype(np.float16)
    k = (rng.standard_normal((batch, q_len * kvh, hd)) * 3).astype(np.float16)
    lens = np.array([0, 17, 39], np.int32)  # the last one runs past the table (row left as is)
    say(f"rope past={past} tables {table_dims}-d")
    qd, kd = torch.from_numpy(q).to(hip_device), torch.from_numpy(k).to(hip_device)
    shape = sin.shape if table_dims == 2 else (1, 1) + sin.shape
    attention_forward_rope_stage_v2_py(qd, kd, torch.from_numpy(sin).view(shape).to(hip_device),
                                       torch.from_numpy(cos).view(shape).to(hip_device), q_len,
                                       batch, heads, kvh, hd, past,
                                       torch.from_numpy(lens).to(hip_device))
    torch.cuda.synchronize()
    qr = A.rope(q, sin, cos, heads, past, lens)
    kr = A.rope(k, sin, cos, kvh, past, lens)
    assert np.array_equal(qd.cpu().numpy().view(np.uint16), qr.view(np.uint16))
    assert np.array_equal(kd.cpu().numpy().view(np.uint16), kr.view(np.uint16))


def test_rope_and_cache_bit_exact(hip_device):
    """The fused decode-step op equals rope on q and k, reshape_and_cache of
    the rotated k and of v, and context lengths = positions + 1."""
    bs, heads, kvh, hd = flags.BLOCK_SIZE, 8, 4, 128
    seqs, nblocks, mb = 5, 20, 4
    info = BlockInfo(head_dim=hd, num_key_value_heads=kvh)
    holder = LayerBlocksHolder.create_contigious_cacher(info, nblocks, hip_device)
    kt, vt = holder.contigious_kv_tenosr
    kt.zero_()
    vt.zero_()
    rng = np.random.default_rng(31)
    sin, cos = A.rope_tables(3 * bs, hd)
    q = (rng.standard_normal((seqs, heads, hd)) * 2).astype(np.float16)
    k = (rng.standard_normal((seqs, kvh, hd)) * 2).astype(np.float16)
    v = rng.standard_normal((seqs, kvh, hd)).astype(np.float16)
    # the fourth position is past the sin/cos table, the fifth past the block table
    pos = np.array([0, 7, bs + 3, 3 * bs + 1, mb * bs + 2], np.int32)
    tables = rng.permutation(nblocks)[:seqs * mb].reshape(seqs, mb).astype(np.int32)
    lens = torch.full((seqs,), -7, dtype=torch.int32, device=hip_device)
    qd, kd, vd = (torch.from_numpy(a).to(hip_device) for a in (q, k, v))
    say("rope_and_cache (tables [1, 1, P, hd])")
    holder.rope_and_cache(qd, kd, vd, torch.from_numpy(sin)[None, None].to(hip_device),
                          torch.from_numpy(cos)[None, None].to(hip_device),
                          torch.from_numpy(pos).to(hip_device),
                          torch.from_numpy(tables).to(hip_device), lens)
    torch.cuda.synchronize()
    q_ref = A.rope(q.reshape(seqs, 1 * heads, hd), sin, cos, heads, -1, pos).reshape(q.shape)
    k_ref = A.rope(k.reshape(seqs, 1 * kvh, hd), sin, cos, kvh, -1, pos).reshape(k.shape)
    kc, vc = A.empty_cache(nblocks, kvh, hd, bs, fill=0.0)
    slots = np.array([tables[s, p // bs] * bs + p % bs if p // bs < mb else -1
                      for s, p in enumerate(pos)], np.int64)
    A.reshape_and_cache(k_ref, v, kc, vc, slots)
    assert np.array_equal(qd.cpu().numpy().view(np.uint16), q_ref.view(np.uint16))
    assert np.array_equal(kd.cpu().numpy().view(np.uint16), k_ref.view(np.uint16))
    assert np.array_equal(kt.cpu().numpy().view(np.uint16), kc.view(np.uint16))
    assert np.array_equal(vt.cpu().numpy().view(np.uint16), vc.view(np.uint16))
    assert lens.cpu().tolist() == (pos + 1).tolist()
    say("rope_and_cache rejects context_lens_out aliasing positions")
    posd = torch.from_numpy(pos).to(hip_device)
    with pytest.raises(ValueError):
        holder.rope_and_cache(qd, kd, vd, torch.from_numpy(sin).to(hip_device),
                              torch.from_numpy(cos).to(hip_device), posd,
                              torch.from_numpy(tables).to(hip_device), posd)
    st = _lib.load().dw4_rope_and_cache(
        seqs, heads, kvh, hd, bs, qd.data_ptr(), heads * hd, kd.data_ptr(), kvh * hd,
        vd.data_ptr(), kvh * hd, torch.from_numpy(sin).to(hip_device).data_ptr(),
        torch.from_numpy(cos).to(hip_device).data_ptr(), sin.shape[0], posd.data_ptr(),
        torch.from_numpy(tables).to(hip_device).data_ptr(), mb,
        holder.layer_key_ptr_table_device.data_ptr(), holder.layer_val_ptr_table_device.data_ptr(),
        info.head_stride, posd.data_ptr() + 4, None)
    assert st == _lib.DW4_ERR_INVALID_ARG

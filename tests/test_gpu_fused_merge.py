"""The fused split merge of short-span decode: a one-token launch of the MFMA
kernels over at most 8 splits merges inside its own launch (the last
work-group of each head group to finish merges the group's splits). A
session batch of 16 tokens over the same short spans runs as one launch whose
merge is the separate merge kernel (every token's span gives the smallest
split size, so all share one split grid), so each one-token call must give
its batch token's bits exactly, and both stay within the oracle's bound.
The calls run back to back on one cache over different head groups and
split counts: a count left non-zero by one launch would make the next
launch merge early or never."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, say

pytestmark = pytest.mark.gpu

CASES = (  # (config, layer, n_seq): the spans are short enough for 4 to 8 splits
    ("B", 0, 512),  # head_dim 64, 8 KV heads in pairs, 4 splits
    ("C", 0, 2048),  # head_dim 256, one KV head, a 512-key window: 4 or 5 splits
    ("A", 0, 512),  # F32, head_dim 256, 8 splits
    ("E", 0, 1024),  # head_dim 256, 4 KV heads in pairs, 8 splits
    ("D", 0, 1000),  # head_dim 128, 8 splits
)


@pytest.mark.parametrize("key,layer,n_seq", CASES)
def test_fused_merge_matches_merge_kernel(orc, key, layer, n_seq):
    cfg = synth.CONFIGS[key]
    window = cfg.layer_window(layer)
    rows = cfg.layer_rows(layer, n_seq, 16)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    pos0 = n_seq - 16
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    with nh.KVCache([rows], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
        kv.append(0, 0, K, V)
        say(f"case fused merge {key}: 16-token batch {pos0}+16 (merge kernel)")
        batch = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        want = orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
        ea, _ = errors(batch, want)
        say(f"  batch max-abs vs oracle {ea:.3e}")
        assert ea <= cfg.tol
        for t in (15, 0, 9, 15):
            say(f"case fused merge {key}: one-token call at {pos0 + t}")
            one = kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, **kw)
            assert np.array_equal(one.view(np.uint32), batch[t:t + 1].view(np.uint32)), t


def test_fused_merge_back_to_back_over_shapes(orc):
    """Alternating decode calls of two layers of different shapes on one cache
    (Llama-3.2-1B at 512 keys, Qwen3-4B at 1000 keys: different head groups,
    4 and 8 splits), and a long span between them that takes the merge
    kernel; each call's bits equal a fresh cache's."""
    cb, cd = synth.CONFIGS["B"], synth.CONFIGS["D"]
    nb, nd, n_long = 512, 1000, 8192
    Kb, Vb = synth.cache_buffer(cb, 0, nb, nb)
    Kd, Vd = synth.cache_buffer(cd, 0, n_long, n_long)
    kwb = dict(n_head=cb.n_head, n_kv=cb.n_kv, head_dim=cb.head_dim, scale=cb.attn_scale)
    kwd = dict(n_head=cd.n_head, n_kv=cd.n_kv, head_dim=cd.head_dim, scale=cd.attn_scale)
    qb = synth.qk_rows(cb, 0, 0, np.arange(nb - 1, nb), cb.n_head)
    qd = synth.qk_rows(cd, 0, 0, np.arange(nd - 1, nd), cd.n_head)
    ql = synth.qk_rows(cd, 0, 0, np.arange(n_long - 1, n_long), cd.n_head)
    calls = [(0, qb, nb, kwb), (1, qd, nd, kwd), (1, ql, n_long, kwd)] * 3
    ref = {}
    for buf, qq, n, kw in calls[:3]:
        with nh.KVCache([nb, n_long], [cb.kv_dim, cd.kv_dim]) as fresh:
            fresh.append(0, 0, Kb, Vb)
            fresh.append(1, 0, Kd, Vd)
            ref[(buf, n)] = fresh.attend(buf, qq, pos0=n - 1, n_seq=n, **kw)
    want_b = orc.attend_layer(qb, Kb, Vb, kv_bf16=True, rows=nb, pos0=nb - 1, n_seq=nb, **kwb)
    want_d = orc.attend_layer(qd, Kd, Vd, kv_bf16=True, rows=n_long, pos0=nd - 1, n_seq=nd, **kwd)
    assert errors(ref[(0, nb)], want_b)[0] <= cb.tol
    assert errors(ref[(1, nd)], want_d)[0] <= cd.tol
    with nh.KVCache([nb, n_long], [cb.kv_dim, cd.kv_dim]) as kv:
        kv.append(0, 0, Kb, Vb)
        kv.append(1, 0, Kd, Vd)
        for i, (buf, qq, n, kw) in enumerate(calls):
            say(f"case fused merge back to back: call {i}, buffer {buf}, span {n}")
            got = kv.attend(buf, qq, pos0=n - 1, n_seq=n, **kw)
            assert np.array_equal(got.view(np.uint32), ref[(buf, n)].view(np.uint32)), i

"""A seeded sweep of batches on the prefill kernels (BF16 caches with V's fp16
copy, the default) against the oracle: head_dim 64, 128 and 256, GQA groups
1 to 8, plain buffers of any row count and rings sized by nnc's rule
(reference model.cpp:1936-1957), causal spans with and without a window,
batches that start and end mid-way through the copy's 32-row groups.
Bound: 5e-3 max-abs, the BF16 tolerance."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, say

pytestmark = pytest.mark.gpu


def _cases(n: int, seed: int = 2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hd = int(rng.choice([64, 128, 256]))
        group = int(rng.choice([1, 2, 4, 8]))
        n_kv = int(rng.choice([1, 2, 4]))
        n_tok = int(rng.integers(17, 300))
        window = int(rng.choice([0, 0, int(rng.integers(40, 700))]))
        n_seq = int(rng.integers(n_tok, 3000))
        if window > 0 and rng.random() < 0.5:
            rows = nh.kv_rows(n_seq + 256, window, n_tok)  # a ring (a multiple of 256 rows)
        else:
            rows = n_seq + int(rng.integers(0, 40))  # a plain buffer, any row count
        out.append((i, hd, group, n_kv, n_tok, window, n_seq, rows))
    return out


@pytest.mark.parametrize("case", _cases(16), ids=lambda c: f"c{c[0]}-hd{c[1]}-g{c[2]}-w{c[5]}")
def test_prefill_sweep(orc, case):
    i, hd, group, n_kv, n_tok, window, n_seq, rows = case
    cfg = synth.AttnConfig(20 + i, f"sweep {i}", group * n_kv, n_kv, hd, 1, window=window, swa_period=2)
    pos0 = n_seq - n_tok
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=n_kv, head_dim=hd, scale=cfg.attn_scale)
    say(f"case sweep {i}: hd {hd} group {group} n_kv {n_kv}, {n_tok} tokens at {pos0}, n_seq {n_seq}, "
        f"rows {rows}, window {window}")
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= 5e-3

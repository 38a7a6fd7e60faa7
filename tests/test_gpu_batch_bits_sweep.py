"""A seeded sweep of session batches (2 to 16 tokens, nnc's batch sizes:
reference model.h:330, session.cpp:340) whose every token must have the bits
of its one-token call (reference src/appnnc/tests.cpp:2631-2661): head_dim 64,
128 and 256, query groups 1 to 8, one to eight KV heads (odd counts take one
KV head per work-group, even ones two), BF16 and F32 caches, plain buffers of
any row count and rings sized by nnc's rule (reference model.cpp:1936-1957),
causal spans with and without a window, batches that start anywhere from the
first position on. Each case also stays within the oracle's bound (BF16
5e-3, F32 1e-3) and prints its parameters before its GPU calls."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import say

pytestmark = pytest.mark.gpu


def _cases(n: int, seed: int = 4096):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hd = int(rng.choice([64, 128, 256]))
        group = int(rng.choice([1, 2, 4, 8]))
        n_kv = int(rng.choice([1, 2, 3, 4, 8]))
        bf16 = bool(rng.random() < 0.75)
        n_tok = int(rng.integers(2, 17))
        window = int(rng.choice([0, 0, int(rng.integers(16, 1200))]))
        pos0 = int(rng.choice([0, int(rng.integers(1, 64)), int(rng.integers(64, 4000)), int(rng.integers(4000, 20000))]))
        n_seq = pos0 + n_tok
        if window > 0 and rng.random() < 0.5:
            rows = nh.kv_rows(n_seq + 512, window, 16)  # a ring (a multiple of 256 rows)
        else:
            rows = n_seq + int(rng.integers(0, 40))  # a plain buffer, any row count
        out.append((i, hd, group, n_kv, bf16, n_tok, window, pos0, rows))
    return out


@pytest.mark.parametrize("case", _cases(24),
                         ids=lambda c: f"c{c[0]}-hd{c[1]}-g{c[2]}-kv{c[3]}-{'bf16' if c[4] else 'f32'}-n{c[5]}")
def test_batch_bits_sweep(orc, case):
    i, hd, group, n_kv, bf16, n_tok, window, pos0, rows = case
    cfg = synth.AttnConfig(40 + i, f"bits sweep {i}", group * n_kv, n_kv, hd, 1, kv_bf16=bf16,
                           tol=5e-3 if bf16 else 1e-3)
    n_seq = pos0 + n_tok
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, causal=True, n_head=cfg.n_head, n_kv=n_kv, head_dim=hd, scale=cfg.attn_scale)
    say(f"case bits sweep {i}: hd {hd} group {group} n_kv {n_kv} {'BF16' if bf16 else 'F32'}, "
        f"{n_tok} tokens at {pos0}, rows {rows}, window {window}")
    with nh.KVCache([rows], [cfg.kv_dim], bf16=bf16) as kv:
        kv.append(0, 0, K, V)
        batch = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        single = np.stack([kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, **kw)[0]
                           for t in range(n_tok)])
    differ = [t for t in range(n_tok) if not np.array_equal(batch[t].view(np.uint32), single[t].view(np.uint32))]
    assert not differ, f"tokens whose batch bits differ from their one-token call: {differ}"
    want = orc.attend_layer(q, K, V, kv_bf16=bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    err = float(np.abs(batch.astype(np.float64) - want).max())
    say(f"  bitwise equal; max-abs vs oracle {err:.3e}")
    assert err <= cfg.tol


def _exact_cases(n: int, seed: int = 8192):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        hd = int(rng.choice([64, 128, 256]))
        group = int(rng.choice([1, 2, 4, 8]))
        n_kv = int(rng.choice([1, 2, 3, 4]))
        bf16 = bool(rng.random() < 0.75)
        n_tok = int(rng.integers(17, 160))
        window = int(rng.choice([0, int(rng.integers(16, 1200))]))
        pos0 = int(rng.choice([0, int(rng.integers(1, 4000)), int(rng.integers(4000, 12000))]))
        n_seq = pos0 + n_tok
        if window > 0 and rng.random() < 0.5:
            rows = nh.kv_rows(n_seq + 512, window, n_tok)
        else:
            rows = n_seq + int(rng.integers(0, 40))
        out.append((i, hd, group, n_kv, bf16, n_tok, window, pos0, rows))
    return out


@pytest.mark.parametrize("case", _exact_cases(8),
                         ids=lambda c: f"x{c[0]}-hd{c[1]}-g{c[2]}-kv{c[3]}-{'bf16' if c[4] else 'f32'}-n{c[5]}")
def test_exact_mode_bits_sweep(orc, case):
    """Batches past a session's 16 tokens in exact mode
    (nnc_hip_kv_set_exact_batches): every token bit for bit against its
    one-token call, as nnc's CPU path gives any batch (reference
    model.cpp:1724-1729)."""
    i, hd, group, n_kv, bf16, n_tok, window, pos0, rows = case
    cfg = synth.AttnConfig(60 + i, f"exact sweep {i}", group * n_kv, n_kv, hd, 1, kv_bf16=bf16,
                           tol=5e-3 if bf16 else 1e-3)
    n_seq = pos0 + n_tok
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, causal=True, n_head=cfg.n_head, n_kv=n_kv, head_dim=hd, scale=cfg.attn_scale)
    say(f"case exact sweep {i}: hd {hd} group {group} n_kv {n_kv} {'BF16' if bf16 else 'F32'}, "
        f"{n_tok} tokens at {pos0}, rows {rows}, window {window}")
    with nh.KVCache([rows], [cfg.kv_dim], bf16=bf16) as kv:
        kv.append(0, 0, K, V)
        kv.set_exact_batches(True)
        batch = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        single = np.stack([kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, **kw)[0]
                           for t in range(n_tok)])
    differ = [t for t in range(n_tok) if not np.array_equal(batch[t].view(np.uint32), single[t].view(np.uint32))]
    assert not differ, f"tokens whose batch bits differ from their one-token call: {differ[:20]}"
    want = orc.attend_layer(q, K, V, kv_bf16=bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    err = float(np.abs(batch.astype(np.float64) - want).max())
    say(f"  bitwise equal; max-abs vs oracle {err:.3e}")
    assert err <= cfg.tol

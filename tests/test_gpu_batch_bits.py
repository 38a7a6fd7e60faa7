"""A token's attention has the same bits in a batch of up to 16 tokens as in a
one-token call (decode), through the C ABI.

nnc runs every forward pass of a session in batches of at most 16 tokens
(MODEL_PREFILL_BATCH, reference src/libnnc/model.h:330; session.cpp:340), MTP
verification batches included (session.cpp:513-578), and checks for its own
CPU path that each token of a batch gets the bits a one-token pass gives it
(src/appnnc/tests.cpp:2631-2661, F32 and BF16 K/V): speculative decoding keeps
a draft only where the batch reproduces plain decoding exactly. Each case here
also stays within the parity bound of the oracle. Each test prints its case
before the GPU calls."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

pytestmark = pytest.mark.gpu

G8 = synth.AttnConfig(9, "group8", 32, 4, 128, 1)  # 2 tokens per work-group
G1 = synth.AttnConfig(10, "group1", 8, 8, 64, 1)  # 16 tokens per work-group

CASES = [
    # (config, layer, first position, batch)
    (synth.CONFIGS["D"], 0, 4000, 16),  # Qwen3-4B, hd 128, group 4: four launches' worth of tokens in one
    (synth.CONFIGS["D"], 1, 8185, 16),  # spans cross 8192 keys: two split sizes, two launches
    (synth.CONFIGS["D"], 2, 0, 5),  # a prompt's first tokens: one-key spans upward
    (synth.CONFIGS["C"], 0, 3000, 16),  # Gemma-3-1B local layer: window 512 in a ring, hd 256
    (synth.CONFIGS["C"], 5, 2047, 9),  # Gemma-3-1B global layer
    (synth.CONFIGS["E"], 0, 2500, 16),  # Gemma-3-4B local layer: window 1024, group 2
    (synth.CONFIGS["B"], 0, 700, 7),  # Llama shape, hd 64
    (synth.CONFIGS["A"], 0, 1000, 16),  # F32 K/V
    (G8, 0, 3000, 16),
    (G1, 0, 1500, 16),
    # batches across a change of split size where short spans take splits of
    # one wavefront chunk (one-token split at the first span, a longer one at
    # the last)
    (synth.CONFIGS["D"], 3, 4088, 16),  # 64-key splits up to 4096 keys, 128 after
    (synth.CONFIGS["B"], 1, 4090, 16),  # hd 64: 64 -> 128
    (synth.CONFIGS["C"], 11, 4090, 9),  # hd 256, one KV head: 32 -> 64
    (synth.CONFIGS["A"], 1, 2040, 16),  # F32 hd 256: 16 -> 32
]


@pytest.mark.parametrize("cfg,layer,pos0,n", CASES, ids=[f"{c.name}-{l}-{p}+{n}" for c, l, p, n in CASES])
def test_batch_matches_one_token_calls_bitwise(orc, cfg, layer, pos0, n):
    n_seq = pos0 + n
    window = cfg.layer_window(layer)
    rows = cfg.layer_rows(layer, n_seq, 16)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, causal=True, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    print(f"case {cfg.name} layer {layer}: tokens {pos0}+{n}, rows {rows}, window {window}", flush=True)
    with nh.KVCache([rows], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
        kv.append(0, 0, K, V)
        batch = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        single = np.stack([kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, **kw)[0]
                           for t in range(n)])
    differ = [t for t in range(n) if not np.array_equal(batch[t].view(np.uint32), single[t].view(np.uint32))]
    assert not differ, f"tokens whose batch bits differ from their one-token call: {differ}"
    want = orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    err = float(np.abs(batch.astype(np.float64) - want).max())
    print(f"  bitwise equal; max-abs vs oracle {err:.3e}", flush=True)
    assert err <= cfg.tol


EXACT_CASES = [
    # (config, layer, first position, batch): batches past 16 tokens in exact mode
    (synth.CONFIGS["D"], 0, 3584, 512),  # Qwen3-4B: the last 512-token chunk of a 4096 prompt
    (synth.CONFIGS["C"], 0, 5000, 300),  # Gemma-3-1B local layer: ring, window 512
    (synth.CONFIGS["E"], 5, 2000, 64),  # Gemma-3-4B global layer, hd 256, group 2
    (synth.CONFIGS["A"], 0, 1000, 40),  # F32 K/V
]


@pytest.mark.parametrize("cfg,layer,pos0,n", EXACT_CASES, ids=[f"{c.name}-{l}-{p}+{n}" for c, l, p, n in EXACT_CASES])
def test_exact_mode_long_batch_matches_one_token_calls_bitwise(orc, cfg, layer, pos0, n):
    """With nnc_hip_kv_set_exact_batches, a chunk of n_batch tokens (nnc's
    prompt chunks, reference tests.cpp:2607) gives every token the bits of its
    one-token call, as nnc's CPU path does (model.cpp:1724-1729); the default
    mode's prefill kernel stays within the parity bound instead."""
    n_seq = pos0 + n
    window = cfg.layer_window(layer)
    rows = cfg.layer_rows(layer, n_seq, n)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, causal=True, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    print(f"case exact mode {cfg.name} layer {layer}: tokens {pos0}+{n}, rows {rows}, window {window}", flush=True)
    with nh.KVCache([rows], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
        kv.append(0, 0, K, V)
        fast = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        kv.set_exact_batches(True)
        batch = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        single = np.stack([kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, **kw)[0]
                           for t in range(n)])
    differ = [t for t in range(n) if not np.array_equal(batch[t].view(np.uint32), single[t].view(np.uint32))]
    assert not differ, f"tokens whose batch bits differ from their one-token call: {differ[:20]}"
    want = orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    err = float(np.abs(batch.astype(np.float64) - want).max())
    err_fast = float(np.abs(fast.astype(np.float64) - want).max())
    print(f"  bitwise equal; max-abs vs oracle {err:.3e} (default mode {err_fast:.3e})", flush=True)
    assert err <= cfg.tol and err_fast <= cfg.tol

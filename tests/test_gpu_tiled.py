"""The tiled fp32-MFMA kernel: batches of more than 16 tokens over F32 caches
and over head shapes outside the MFMA kernels' (head_dim a multiple of 16 up
to 512). Each case against the oracle within the F32 (1e-3) or BF16 (5e-3)
bound: nnc's embedding call (reference model.cpp:2355-2368: the whole input
in one batch, F32, bidirectional, local layers over a symmetric window) at
EmbeddingGemma-300M's shape, causal F32 chunks over a wrapped ring, a gated
BF16 batch at head_dim 80, row blocks that end mid-token (group 3), one
split and many, and the no-alloc entry point with the partials in the fixed
scratch (bits equal to attend_device)."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import hip_rt, synth

from gpu_util import errors, say

pytestmark = pytest.mark.gpu

EMB = synth.AttnConfig(5, "embeddinggemma-300m", 3, 1, 256, 24, kv_bf16=False, window=512, swa_period=6, tol=1e-3)


@pytest.mark.parametrize("layer,n", ((0, 700), (5, 700), (0, 77)))
def test_embedding_call(orc, layer, n):
    """One bidirectional batch of the whole input (local layer 0: +-256
    keys; global layer 5: every key)."""
    cfg = EMB
    window = cfg.layer_window(layer)
    K, V = synth.cache_buffer(cfg, layer, n, n)
    q = synth.qk_rows(cfg, layer, 0, np.arange(n), cfg.n_head)
    kw = dict(window=window, causal=False, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    say(f"case tiled embedding layer {layer} (window {window}), {n} tokens")
    with nh.KVCache([n], [cfg.kv_dim], bf16=False) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=0, n_seq=n, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=False, rows=n, pos0=0, n_seq=n, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= 1e-3


@pytest.mark.parametrize("key,layer,n_seq,pos0,n_tok", (
    ("A", 0, 3000, 2000, 1000),  # F32, head_dim 256, group 4: many splits
    ("A", 0, 200, 100, 100),  # one split
    ("C", 0, 3000, 2900, 100),  # an F32 sliding layer: a 768-row ring, wrapped
))
def test_f32_causal_chunks(orc, key, layer, n_seq, pos0, n_tok):
    base = synth.CONFIGS[key]
    cfg = synth.AttnConfig(base.index, base.name, base.n_head, base.n_kv, base.head_dim, base.n_layer, kv_bf16=False,
                           window=base.window, swa_period=base.swa_period, tol=1e-3)
    window = cfg.layer_window(layer)
    rows = cfg.layer_rows(layer, n_seq, 128)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case tiled F32 {key}: rows {rows} window {window} tokens {pos0}+{n_tok}")
    with nh.KVCache([rows], [cfg.kv_dim], bf16=False) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=pos0 + n_tok, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=False, rows=rows, pos0=pos0, n_seq=pos0 + n_tok, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= 1e-3


def test_bf16_generic_shape_with_gate(orc):
    """head_dim 80, 24 query heads over 8 KV heads (group 3: a 64-row block
    ends mid-token), 300 tokens, Qwen3.5's output gate."""
    cfg = synth.AttnConfig(12, "hd80 g3", 24, 8, 80, 1)
    n_seq, pos0, n_tok = 1500, 1200, 300
    K, V = synth.cache_buffer(cfg, 0, n_seq, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    gate = np.random.default_rng(5).standard_normal(q.shape).astype(np.float32)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=80, scale=cfg.attn_scale)
    say("case tiled BF16 head_dim 80, group 3, gated, 300 tokens")
    with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=pos0 + n_tok, gate=gate, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=n_seq, pos0=pos0, n_seq=pos0 + n_tok, **kw)
    want = want / (1.0 + np.exp(-gate.astype(np.float64)))
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e}")
    assert ea <= 5e-3


def test_tiled_noalloc_matches_attend_device(orc):
    """A 200-token F32 batch through nnc_hip_attend_device_noalloc (partials
    in the library's fixed array) gives attend_device's bits."""
    cfg = synth.CONFIGS["A"]
    n_seq, pos0, n_tok = 1024, 824, 200
    K, V = synth.cache_buffer(cfg, 0, n_seq, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    with nh.KVCache([n_seq], [cfg.kv_dim], bf16=False) as kv:
        kv.append(0, 0, K, V)
        q_dev, o_a, o_b = hip_rt.malloc(q.nbytes), hip_rt.malloc(q.nbytes), hip_rt.malloc(q.nbytes)
        try:
            hip_rt.to_device(q_dev, q)
            say("case tiled F32 200 tokens: attend_device and the no-alloc form")
            kv.attend_device(0, q_dev, o_a, n_tok=n_tok, pos0=pos0, **kw)
            kv.attend_device_noalloc(0, q_dev, o_b, n_tok=n_tok, pos0=pos0, **kw)
            kv.sync()
            a = hip_rt.to_host(np.empty_like(q), o_a)
            b = hip_rt.to_host(np.empty_like(q), o_b)
        finally:
            for d in (q_dev, o_a, o_b):
                hip_rt.free(d)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    want = orc.attend_layer(q, K, V, kv_bf16=False, rows=n_seq, pos0=pos0, n_seq=pos0 + n_tok, **kw)
    assert errors(a, want)[0] <= 1e-3

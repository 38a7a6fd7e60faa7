"""The benchmark configurations at their full spans, ring buffers against full
buffers bit for bit, a prefill-then-decode session, the query-group sizes the
models do not use, F32 decode at every head size, and sharp score
distributions, through the C ABI against the oracle (itself pinned against
the reference in test_oracle.py).

Bounds: max-abs 5e-3 for BF16 K/V and 1e-3 for F32 (nnc's CPU output as the
reference), and where outputs grow large, 5e-3 * (1 + |ref|) per element.
Each test prints its case before the GPU calls."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, run_case, say

pytestmark = pytest.mark.gpu


def check(got, want, tol, label):
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= tol, (label, ea)


# ---- the configurations' full spans -----------------------------------------------------

@pytest.mark.parametrize("layer", (0, 9))
def test_llama_decode_at_16k(orc, layer):
    """B: Llama-3.2-1B decode at its longest context, 16384 keys."""
    cfg = synth.CONFIGS["B"]
    got, want = run_case(orc, cfg, layer, n_seq=16384, pos0=16383, n_tok=1)
    check(got, want, cfg.tol, ("B", layer))


@pytest.mark.parametrize("layer,rows", ((5, None), (0, None)))
def test_gemma3_1b_last_prefill_chunk(orc, layer, rows):
    """C: the last 2048-token chunk of an 8192-token prompt (keys up to 8191)
    on the global layer 5 (8192 rows) and the local layer 0 (a ring of 2560
    rows, window 512)."""
    cfg = synth.CONFIGS["C"]
    got, want = run_case(orc, cfg, layer, n_seq=8192, pos0=6144, n_tok=2048, n_batch=2048, rows=rows)
    check(got, want, cfg.tol, ("C", layer))


@pytest.mark.parametrize("layer,rows", ((5, 16640), (0, None)))
def test_gemma3_4b_last_prefill_chunk(orc, layer, rows):
    """E: the last 1024-token chunk of a 16384-token prompt on a global layer
    (16640 rows: the prompt and 256 decode steps; group 2, head_dim 256) and on
    a local layer (window 1024, a ring of 2048 rows)."""
    cfg = synth.CONFIGS["E"]
    got, want = run_case(orc, cfg, layer, n_seq=16384, pos0=15360, n_tok=1024, n_batch=1024, rows=rows)
    check(got, want, cfg.tol, ("E", layer))


@pytest.mark.parametrize("layer", (5, 0))
def test_gemma3_4b_session_prefill_then_decode(orc, layer):
    """E as a session runs it: three 1024-token chunks appended and attended
    in turn, then ten decode steps, each appending its row first; every call
    checked against the oracle on the buffer as it stands."""
    cfg = synth.CONFIGS["E"]
    chunk, n_prompt, n_dec = 1024, 3072, 10
    n_ctx = n_prompt + n_dec
    window = cfg.layer_window(layer)
    rows = cfg.layer_rows(layer, n_ctx, chunk)
    k, v = synth.kv_rows_f32(cfg, layer, np.arange(n_ctx))
    q = synth.qk_rows(cfg, layer, 0, np.arange(n_ctx), cfg.n_head)
    K = np.zeros((rows, cfg.kv_dim), np.uint16)  # the host mirror of the device buffer
    V = np.zeros_like(K)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    steps = [(p, chunk) for p in range(0, n_prompt, chunk)] + [(n_prompt + i, 1) for i in range(n_dec)]
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        for pos0, n in steps:
            say(f"case E session layer {layer} rows {rows}: tokens {pos0}+{n}")
            kv.append_f32(0, pos0, k[pos0:pos0 + n], v[pos0:pos0 + n])
            r = np.arange(pos0, pos0 + n) % rows
            K[r] = nh.bf16_round(k[pos0:pos0 + n])
            V[r] = nh.bf16_round(v[pos0:pos0 + n])
            got = kv.attend(0, q[pos0:pos0 + n], pos0=pos0, n_seq=pos0 + n, **kw)
            want = orc.attend_layer(q[pos0:pos0 + n], K, V, kv_bf16=True, rows=rows, pos0=pos0, n_seq=pos0 + n, **kw)
            check(got, want, cfg.tol, (layer, pos0))


# ---- ring against full buffer -----------------------------------------------------------

def test_ring_matches_full_buffer_bitwise():
    """A sliding layer's ring gives exactly what a full buffer gives, through
    many wraps, a step back and a rewind to 0 (reference tests.cpp:2595-2629:
    window 40, batches of 16 -> a 256-row ring against 1200 rows; forward
    0..700 by 16, 700..720 by 1, back to 705 and on to 760 by 16, back to 0
    and on to 300 by 16). Each pass writes fresh rows, as new tokens would."""
    cfg = synth.AttnConfig(9, "ring", 4, 2, 64, 1, window=40, swa_period=6)
    rows = nh.kv_rows(1200, 40, 16)
    assert rows == 256 and nh.max_rewind(rows, 40) == 216
    kw = dict(window=40, n_head=4, n_kv=2, head_dim=64, scale=0.125)
    n_cmp = 0
    with nh.KVCache([rows, 1200], [cfg.kv_dim, cfg.kv_dim]) as kv:
        for pas, (a, b, step) in enumerate(((0, 700, 16), (700, 720, 1), (705, 760, 16), (0, 300, 16))):
            say(f"case ring pass {pas}: positions {a}..{b} by {step}")
            pcfg = synth.AttnConfig(20 + pas, "ring", 4, 2, 64, 1)  # fresh rows per pass
            k, v = synth.kv_rows_f32(pcfg, 0, np.arange(b))
            q = synth.qk_rows(pcfg, 0, 0, np.arange(b), 4)
            for p in range(a, b, step):
                n = min(step, b - p)
                for buf in (0, 1):
                    kv.append_f32(buf, p, k[p:p + n], v[p:p + n])
                ring = kv.attend(0, q[p:p + n], pos0=p, n_seq=p + n, **kw)
                full = kv.attend(1, q[p:p + n], pos0=p, n_seq=p + n, **kw)
                assert np.array_equal(ring.view(np.uint32), full.view(np.uint32)), (pas, p)
                n_cmp += 1
    say(f"  {n_cmp} calls bitwise equal")


# ---- group sizes, F32 head sizes --------------------------------------------------------

G1 = synth.AttnConfig(10, "group1", 8, 8, 64, 1)
G8 = synth.AttnConfig(11, "group8", 32, 4, 128, 1)
G8W = synth.AttnConfig(12, "group8 hd256", 16, 2, 256, 1)


@pytest.mark.parametrize("cfg", (G1, G8, G8W), ids=lambda c: c.name)
def test_prefill_groups_1_and_8(orc, cfg):
    """Batches above 16 tokens (the prefill kernel) at query groups 1 and 8."""
    got, want = run_case(orc, cfg, 0, n_seq=1500, pos0=1200, n_tok=300, n_batch=300)
    check(got, want, cfg.tol, cfg.name)


F32_64 = synth.AttnConfig(13, "f32 hd64", 8, 2, 64, 1, kv_bf16=False, tol=1e-3)
F32_128 = synth.AttnConfig(14, "f32 hd128", 16, 4, 128, 1, kv_bf16=False, tol=1e-3)


@pytest.mark.parametrize("cfg", (F32_64, F32_128), ids=lambda c: c.name)
def test_f32_decode_head_sizes(orc, cfg):
    """F32 K/V decode at head_dim 64 and 128 (config A covers 256), one token
    and a 12-token batch."""
    for pos0, n in ((3999, 1), (3988, 12)):
        got, want = run_case(orc, cfg, 0, n_seq=pos0 + n, pos0=pos0, n_tok=n)
        check(got, want, cfg.tol, (cfg.name, n))


# ---- sharp scores -----------------------------------------------------------------------

@pytest.mark.parametrize("n_tok", (1, 16, 200))
def test_peaked_scores(orc, n_tok):
    """Q scaled by 6 (scores spread over tens of units, so few keys carry the
    weight and the running offset moves often): decode, a session batch and the
    prefill kernel, with the bound relative to each output."""
    cfg = synth.CONFIGS["D"]
    n_seq = 3000
    K, V = synth.cache_buffer(cfg, 1, n_seq, n_seq)
    pos0 = n_seq - n_tok
    q = 6.0 * synth.qk_rows(cfg, 1, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case peaked scores, D, {n_tok} tokens")
    with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=n_seq, pos0=pos0, n_seq=n_seq, **kw)
    d = np.abs(got.astype(np.float64) - want)
    say(f"  max-abs {d.max():.3e}; max of d / (1 + |ref|) {(d / (1 + np.abs(want))).max():.3e}")
    assert np.all(d <= cfg.tol * (1.0 + np.abs(want)))
    assert d.max() <= cfg.tol


@pytest.mark.parametrize("n_tok,v_mul", ((1, 100.0), (16, 100.0), (200, 100.0), (200, 1.4)))
def test_large_values(orc, n_tok, v_mul):
    """V scaled up and Q by 6 (peaked weights, scores up to ~90 in log2 units).
    With V x100 (|V| up to about 550) outputs reach a few hundred; there a
    score's own fp32 rounding moves a weight by ~1e-5 and an output by ~1e-3
    in any fp32 implementation, the reference's included, so the bound is
    relative to 1 + |ref| per element: 2.5e-3 for decode and a session batch
    (split-K kernels, every product near-fp32; measured 9.8e-4, while P
    rounded to bf16 alone would give about 8e-3), 5e-3 for the prefill kernel
    (values beyond 8 keep it off V's fp16 copy, so it takes P as bf16 hi +
    lo). With V x1.4 (|V| below 8) the prefill kernel reads the fp16 copy
    with P rounded to fp16, whose error grows with |V|: both of its bounds
    hold."""
    cfg = synth.CONFIGS["D"]
    n_seq = 8192
    K, V = synth.cache_buffer(cfg, 2, n_seq, n_seq)
    V = synth.to_cache_dtype(cfg, v_mul * nh.bf16_to_f32(V))
    pos0 = n_seq - n_tok
    q = 6.0 * synth.qk_rows(cfg, 2, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case V x{v_mul:g} (max |V| {np.abs(nh.bf16_to_f32(V)).max():.1f}), Q x6, D, {n_tok} tokens")
    with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=n_seq, pos0=pos0, n_seq=n_seq, **kw)
    d = np.abs(got.astype(np.float64) - want)
    say(f"  max-abs {d.max():.3e}; max of d / (1 + |ref|) {(d / (1 + np.abs(want))).max():.3e}; "
        f"max |ref| {np.abs(want).max():.1f}")
    rel = 2.5e-3 if n_tok <= 16 else cfg.tol
    assert np.all(d <= rel * (1.0 + np.abs(want)))
    if np.abs(nh.bf16_to_f32(V)).max() <= 8.0:
        assert d.max() <= cfg.tol


@pytest.mark.parametrize("n_tok", (1, 16, 100))
def test_dominant_key_returns_its_value_row(n_tok):
    """Closed form: when every query of a KV head is a large multiple of one
    key j, the other keys' weights are below 2^-149 and vanish, so each output
    row is exactly V[j] of its KV head (bf16 widened to fp32), whatever the
    path (decode, session batch, prefill kernel)."""
    cfg = synth.CONFIGS["D"]
    n_seq, j = 2600, 777
    K, V = synth.cache_buffer(cfg, 2, n_seq, n_seq)
    kf = nh.bf16_to_f32(K).reshape(n_seq, cfg.n_kv, cfg.head_dim)
    # scale * (q . k_j) = 300 for q = c k_j; other keys score at most ~0.3 of that
    c = 300.0 / (cfg.attn_scale * (kf[j] ** 2).sum(axis=-1))  # [n_kv]
    qh = np.repeat((c[:, None] * kf[j])[:, None, :], cfg.group, axis=1)  # [n_kv, group, hd]
    q = np.tile(qh.reshape(1, -1), (n_tok, 1)).astype(np.float32)
    scores = cfg.attn_scale * np.einsum("kd,nkd->nk", kf[j] * c[:, None], kf)
    assert (np.sort(scores, axis=0)[-2] < scores[j] - 160).all()  # exp(-160) < 2^-149
    pos0 = n_seq - n_tok
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case dominant key {j}, D, {n_tok} tokens")
    with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    vj = nh.bf16_to_f32(V[j]).reshape(cfg.n_kv, 1, cfg.head_dim)
    want = np.tile(np.repeat(vj, cfg.group, axis=1).reshape(1, -1), (n_tok, 1))
    assert np.array_equal(got, want)

"""Parity of the HIP attention op against nnc's CPU attention (the oracle,
itself pinned against the reference in test_oracle.py), through the C ABI.

Bounds (max-abs over all outputs): 1e-3 for F32 K/V, 5e-3 for BF16 K/V.
Each test prints its case before the GPU call."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, run_case, say

pytestmark = pytest.mark.gpu


# ---- decode -----------------------------------------------------------------------------

@pytest.mark.parametrize("key,layers,ctx", [
    ("A", (0, 1, 17), 1024),       # Gemma-3-270M: F32 K/V, hd 256, 1024 keys
    ("B", (0, 15), 512),           # Llama-3.2-1B with RoPE NORM, hd 64
    ("B", (3,), 4096),
    ("C", (0, 5), 8192),           # Gemma-3-1B: a local (ring 2560) and a global layer
    ("D", (0,), 4096),             # Qwen3-4B, RMS-normed Q/K, hd 128
    ("E", (0, 5), 16640),          # Gemma-3-4B: local ring (window 1024) and global, g = 2
])
def test_decode_parity(orc, key, layers, ctx):
    cfg = synth.CONFIGS[key]
    for layer in layers:
        got, want = run_case(orc, cfg, layer, n_seq=ctx, pos0=ctx - 1, n_tok=1, n_batch=2048 if key == "C" else 1024)
        ea, er = errors(got, want)
        say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
        assert ea <= cfg.tol, (key, layer, ea)


def test_decode_qwen3_32k_full_size(orc):
    """Config D at its headline context: one layer, 32768 cached keys."""
    cfg = synth.CONFIGS["D"]
    got, want = run_case(orc, cfg, 7, n_seq=32768, pos0=32767, n_tok=1)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= cfg.tol


def test_decode_is_deterministic_and_matches_textbook(orc):
    cfg = synth.CONFIGS["D"]
    n_seq = 3000
    K, V = synth.cache_buffer(cfg, 2, n_seq, n_seq)
    q = synth.qk_rows(cfg, 2, 0, np.array([n_seq - 1]), cfg.n_head)
    kw = dict(n_head=32, n_kv=8, head_dim=128, scale=cfg.attn_scale)
    say("case decode determinism, D, 3000 keys")
    with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        a = kv.attend(0, q, pos0=n_seq - 1, **kw)
        b = kv.attend(0, q, pos0=n_seq - 1, **kw)
    assert np.array_equal(a, b)
    t = orc.textbook(q, K, V, kv_bf16=True, rows=n_seq, pos0=n_seq - 1, **kw)
    assert errors(a, t)[0] <= 5e-4  # the split-Q MFMA scores are near-fp32


def test_decode_edge_spans(orc):
    """One key (position 0), a ring that wraps inside a split, a span that
    starts mid-block, and an empty span (an MTP drafter's query past the
    keys its target evaluated: zeros, the l == 0 rule)."""
    cfg = synth.AttnConfig(7, "edge", 8, 2, 128, 1, window=300, swa_period=6)
    kw = dict(n_head=8, n_kv=2, head_dim=128, scale=0.09)
    rows = 512
    n_seq = 1700  # ring of 512 rows holds positions 1188..1699; row 0 is position 1536
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    with nh.KVCache([rows, 64], [256, 256]) as kv:
        kv.append(0, 0, K, V)
        for pos, n_s, w in ((1699, 1700, 300), (1699, 1700, 512), (1600, 1700, 300), (1650, 1700, 0)):
            say(f"case ring decode pos {pos} window {w}")
            q = synth.qk_rows(cfg, 0, 0, np.array([pos]), 8)
            if w == 0:
                with pytest.raises(nh.NncError) as e:  # keys 0.. are long gone from a 512-row ring
                    kv.attend(0, q, pos0=pos, n_seq=n_s, window=w, **kw)
                assert e.value.status == nh.NncStatus.CONTEXT_FULL
                continue
            got = kv.attend(0, q, pos0=pos, n_seq=n_s, window=w, **kw)
            want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=pos, n_seq=n_s, window=w, **kw)
            assert errors(got, want)[0] <= 5e-3
        # position 0: one key, the output is that key's V row for every head
        k1, v1 = synth.kv_rows_f32(cfg, 0, np.array([0]))
        kv.append_f32(1, 0, k1, v1)
        q = synth.qk_rows(cfg, 0, 0, np.array([0]), 8)
        say("case single key")
        got = kv.attend(1, q, pos0=0, **kw)
        vb = nh.bf16_to_f32(nh.bf16_round(v1)).reshape(2, 128)
        assert np.array_equal(got.reshape(8, 128), np.repeat(vb, 4, axis=0))
        say("case empty span")
        got = kv.attend(1, q, pos0=10, n_seq=5, window=3, **kw)
        assert np.all(got == 0.0)


def test_drafter_reads_target_cache(orc):
    """An MTP drafter attends over its target's cache (kv_ext, reference
    model.cpp:1664, :1707) with n_seq = the target's cur_pos, which can lie
    below the drafter's own position: keys 0 .. n_seq - 1 (causal) or the
    window's part of them."""
    cfg = synth.CONFIGS["D"]
    rows, n_seq = 2048, 1990
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        for pos, window in ((1995, 0), (1992, 700), (1989, 0)):
            say(f"case drafter read pos {pos} n_seq {n_seq} window {window}")
            q = synth.qk_rows(cfg, 0, 0, np.array([pos]), cfg.n_head)
            got = kv.attend(0, q, pos0=pos, n_seq=n_seq, window=window, **kw)
            want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=pos, n_seq=n_seq, window=window, **kw)
            assert errors(got, want)[0] <= cfg.tol


# ---- prefill ----------------------------------------------------------------------------

@pytest.mark.parametrize("key,window", [("D", 0), ("D", 300), ("C", 0), ("C", 512)])
def test_prefill_batch_past_n_seq(orc, key, window):
    """A batch on the prefill kernels whose last tokens sit past n_seq (keys
    end at n_seq - 1 for them, as for a drafter reading its target's cache),
    with and without a window, against the oracle."""
    cfg = synth.CONFIGS[key]
    rows, n_seq, pos0, n_tok = 2048, 1990, 1960, 40
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case prefill past n_seq: {key}, {n_tok} tokens at {pos0}, n_seq {n_seq}, window {window}")
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= cfg.tol

@pytest.mark.parametrize("key,layer,n_seq,chunk", [
    ("D", 0, 4096, 512),    # Qwen3-4B: the last 512-token chunk of a 4096 prompt
    ("D", 1, 512, 512),     # the first chunk: the causal triangle only
    ("C", 0, 6144, 2048),   # Gemma-3-1B local layer: ring 2560, window 512
    ("C", 5, 4096, 2048),   # Gemma-3-1B global layer
    ("E", 0, 3072, 1024),   # Gemma-3-4B local layer: ring 2048, window 1024, g = 2
    ("B", 0, 700, 300),     # Llama shape, hd 64, a ragged chunk
])
def test_prefill_parity(orc, key, layer, n_seq, chunk):
    cfg = synth.CONFIGS[key]
    got, want = run_case(orc, cfg, layer, n_seq=n_seq, pos0=n_seq - chunk, n_tok=chunk, n_batch=chunk)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= cfg.tol, (key, layer, ea)


_EDGE = synth.AttnConfig(7, "edge", 8, 2, 128, 1, window=300, swa_period=6)


@pytest.mark.parametrize("cfg,layer,rows,n_seq,chunk", [
    (synth.CONFIGS["D"], 0, 1000, 1000, 300),   # rows not a multiple of 32: the copy's last group runs past them
    (synth.CONFIGS["B"], 0, 1000, 1000, 389),   # the same at hd 64
    (synth.CONFIGS["C"], 0, 1000, 1000, 300),   # hd 256, window 512: the span starts mid-group
    (_EDGE, 0, 512, 1700, 200),                 # hd 128, window 300, a 512-row ring wrapping mid-span
])
def test_prefill_fp16_copy_groups(orc, cfg, layer, rows, n_seq, chunk):
    """The prefill kernels read V's fp16 copy in whole 32-row groups, from
    the span's first key rounded down to 32 (keys before it masked), up to
    the end of the group of its last key. Spans that start mid-group, end in
    a group past the buffer's rows, and wrap a ring, against the oracle."""
    got, want = run_case(orc, cfg, layer, n_seq=n_seq, pos0=n_seq - chunk, n_tok=chunk, rows=rows)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= cfg.tol, (cfg.name, rows, n_seq, ea)


@pytest.mark.parametrize("key,chunk", [("C", 300), ("D", 200)])
def test_prefill_ring_rows_not_whole_groups(orc, key, chunk):
    """A 1000-row ring (rows not a multiple of 32) whose span wraps: the
    prefill kernels take the bf16 V there (the fp16 copy's groups do not tile
    such a ring). nnc sizes every ring in multiples of 256 rows
    (model.cpp:1936-1957), and the oracle's restatement of its dispatch
    assumes that, so the check is against the double-precision textbook."""
    cfg = synth.AttnConfig(10, f"ring 1000 {key}", synth.CONFIGS[key].n_head, synth.CONFIGS[key].n_kv,
                           synth.CONFIGS[key].head_dim, 1, window=512, swa_period=6)
    rows, n_seq = 1000, 1600
    pos0 = n_seq - chunk
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=512, causal=True, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    say(f"case {cfg.name}: {chunk} tokens at {pos0}, keys wrap the ring")
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.textbook(q, K, V, kv_bf16=True, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= 5e-3


def test_fp16_copy_same_bits_by_any_append():
    """V's fp16 copy is written by whole 32-row slot sets for batches of 16
    rows or more and element by element for fewer; through F32 rows and BF16
    rows (a plain copy, then the copy's own pass). Caches filled in one or
    two appends and in pieces of every kind — ring wraps and groups shared
    with earlier pieces included — must hold the same copy: a prefill batch
    over each gives the same bits."""
    rng = np.random.default_rng(17)
    n_head, n_kv, hd, rows, n = 8, 2, 128, 512, 700
    kv_dim = n_kv * hd
    k = rng.standard_normal((n, kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, kv_dim)).astype(np.float32)
    kb = nh.bf16_round(k)
    vb = nh.bf16_round(v)
    q = rng.standard_normal((100, n_head * hd)).astype(np.float32)
    kw = dict(pos0=600, n_seq=n, window=200, n_head=n_head, n_kv=n_kv, head_dim=hd, scale=0.09)
    pieces = [(0, 1), (1, 1), (2, 37), (39, 5), (44, 300), (344, 17), (361, 3), (364, 336)]
    outs = []
    for label in ("f32 in two", "f32 in pieces", "bf16 in pieces"):
        say(f"case fp16 copy writes: {label}")
        with nh.KVCache([rows], [kv_dim]) as kv:
            if label == "f32 in two":
                kv.append_f32(0, 0, k[:400], v[:400])
                kv.append_f32(0, 400, k[400:], v[400:])
            else:
                for p0, m in pieces:
                    if label.startswith("f32"):
                        kv.append_f32(0, p0, k[p0:p0 + m], v[p0:p0 + m])
                    else:
                        kv.append(0, p0, kb[p0:p0 + m], vb[p0:p0 + m])
            outs.append(kv.attend(0, q, **kw))
    for o in outs[1:]:
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32))


def test_prefill_odd_batches(orc):
    """Batches of 2 and 5 tokens (session-sized: the split-K kernel), 17 and 37
    (the prefill kernel, rows that do not fill a tile), and a bidirectional
    batch (the embedding path's spans) with and without a window."""
    cfg = synth.CONFIGS["D"]
    for n_tok in (2, 5, 17, 37):
        got, want = run_case(orc, cfg, 3, n_seq=900, pos0=900 - n_tok, n_tok=n_tok)
        assert errors(got, want)[0] <= cfg.tol, n_tok
    ecfg = synth.AttnConfig(8, "embed", 4, 1, 256, 1)
    for w in (0, 128):
        n = 300
        K, V = synth.cache_buffer(ecfg, 0, n, n)
        q = synth.qk_rows(ecfg, 0, 0, np.arange(n), 4)
        kw = dict(window=w, causal=False, n_head=4, n_kv=1, head_dim=256, scale=1 / 16)
        say(f"case bidirectional window {w}")
        with nh.KVCache([n], [256]) as kv:
            kv.append(0, 0, K, V)
            got = kv.attend(0, q, pos0=0, n_seq=n, **kw)
        want = orc.attend_layer(q, K, V, kv_bf16=True, rows=n, pos0=0, n_seq=n, **kw)
        assert errors(got, want)[0] <= 5e-3, w


@pytest.mark.parametrize("shape,n,w", (("A", 700, 256), ("D", 300, 0), ("D", 1300, 64)))
def test_f32_embedding_batch(orc, shape, n, w):
    """nnc_embed's attention (reference model.cpp:2368, spans :2308-2315): an
    F32 cache of the whole sequence, every token in one bidirectional batch,
    with a symmetric window or none; F32 bound of the oracle. 1300 tokens
    take two launches (1024 tokens each at most)."""
    base = synth.CONFIGS[shape]
    cfg = synth.AttnConfig(9, f"embed {shape}", base.n_head, base.n_kv, base.head_dim, 1, kv_bf16=False,
                           qk_norm=base.qk_norm)
    K, V = synth.cache_buffer(cfg, 0, n, n)
    q = synth.qk_rows(cfg, 0, 0, np.arange(n), cfg.n_head)
    kw = dict(window=w, causal=False, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    say(f"case F32 embedding {shape}: {n} tokens, window {w}")
    with nh.KVCache([n], [cfg.kv_dim], bf16=False) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=0, n_seq=n, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=False, rows=n, pos0=0, n_seq=n, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
    assert ea <= 1e-3


def test_cache_creation_logs_device_and_bytes():
    """nnc_hip_kv_create reports the device and the device memory it holds at
    INFO through the log callback (the counterpart of nnc's context line)."""
    lines = []
    nh.set_log_callback(lambda level, msg: lines.append((level, msg)))
    try:
        say("case creation log line")
        with nh.KVCache([1024, 512], [1024, 1024]) as kv:
            nbytes = kv.nbytes
    finally:
        nh.set_log_callback(None)
    info = [m for level, m in lines if level == 1]
    say(f"  {info}")
    assert len(info) == 1
    assert "2 K/V buffers" in info[0] and "BF16 K/V" in info[0]
    assert f"{nbytes / 1e6:.1f} MB" in info[0]


def test_prefill_fp16_shadow_and_fallbacks(orc, monkeypatch):
    """BF16 caches keep an fp16 copy of V for the prefill kernel (P in fp16,
    one MFMA per P . V product) holding values up to 8 in magnitude. A V
    value beyond that (10, or 1e5 past fp16's range) sends the prefill through
    the bf16 path (P as bf16 hi + lo against the exact bf16 V), bit for bit
    what a cache without the copies (NNC_HIP_F16_SHADOW=0) gives; a value of 6
    keeps the fp16 path. K is read as bf16 with Q as hi + lo on both paths, so
    large K or Q values need no fallback. Every variant stays within the BF16
    bound of the oracle, and within 5e-3 * (1 + |ref|) where a V of 1e5 makes
    outputs large."""
    cfg = synth.CONFIGS["D"]
    n_seq, n_tok = 1024, 64
    pos0 = n_seq - n_tok
    K, V = synth.cache_buffer(cfg, 0, n_seq, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)

    def run(K, V, q, label, relative=False):
        say(f"case prefill {label}")
        with nh.KVCache([n_seq], [cfg.kv_dim]) as kv:
            kv.append(0, 0, K, V)
            got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
        want = orc.attend_layer(q, K, V, kv_bf16=True, rows=n_seq, pos0=pos0, n_seq=n_seq, **kw)
        d = np.abs(got.astype(np.float64) - want)
        say(f"  max-abs {d.max():.3e}, max |ref| {np.abs(want).max():.3e}")
        if relative:
            assert np.all(d <= cfg.tol * (1.0 + np.abs(want))), label
        else:
            assert d.max() <= cfg.tol, label
        return got, want

    def bits(K, V, label):  # with the copy, then without it
        with_copy, _ = run(K, V, q, label)
        monkeypatch.setenv("NNC_HIP_F16_SHADOW", "0")
        without, _ = run(K, V, q, label + ", no shadow (bf16 K/V, Q hi + lo)")
        monkeypatch.delenv("NNC_HIP_F16_SHADOW")
        return with_copy.view(np.uint32), without.view(np.uint32)

    base, plain = bits(K, V, "fp16 shadow")
    assert not np.array_equal(base, plain)  # the two paths round differently
    for val, copy_used in ((6.0, True), (10.0, False)):  # the copy's limit is 8
        V3 = V.copy()
        V3[200, 9] = nh.bf16_round(np.array([val], np.float32))[0]
        a, b = bits(K, V3, f"cache V value {val:g}")
        assert np.array_equal(a, b) != copy_used, val
    big = nh.bf16_round(np.array([1.0e5], np.float32))[0]  # past fp16's range
    K2 = K.copy()
    K2[100, 5] = big
    run(K2, V, q, "cache K value past fp16 range (no effect on the path)")
    V2 = V.copy()
    V2[200, 9] = big  # KV head 0, element 9: query heads 0..3 see it
    got, want = run(K, V2, q, "cache V value past fp16 range", relative=True)
    assert np.abs(want[:, 9::cfg.head_dim][:, :4]).max() > 10.0  # the value reached the outputs
    q2 = q.copy()
    q2[3, 7] = 1.0e6  # q * scale * log2(e) past fp16's range in one work-group
    run(K, V, q2, "Q value past fp16 range", relative=True)


def test_prefill_fp16_weights_within_their_bound(orc):
    """The fp16 P . V path at its limit, closed form: every query row weighs
    three keys only (unit K rows e0, e1, e2; every other key scores 60 log2
    units lower and weighs 0), with V rows 0, +8 and -8 (the copy's limit),
    scores 20, 20 - a and 20 - b in log2 units for random a, b in [0, 1).
    The kernel's offset sits 8 below the row max, so the max key weighs
    exactly 2^8 and the other two land anywhere in (2^7, 2^8], their fp16
    roundings in either direction (relative error up to 2^-11, just above
    2^7). With the row sum taken from the same rounded weights, an output
    moves by sum_k w_k e_k (V_k - out), so each row must stay within
    2^-11 * sum_k w_k |V_k - out| of the oracle (plus 2e-6 for the
    near-fp32 scores): 1024 rows of a 256-token chunk (the prefill kernel),
    many of them near the worst case."""
    n_head, n_kv, hd, n_seq, n_tok = 4, 1, 128, 1024, 256
    scale = 1.0 / np.sqrt(hd)
    log2e = 1.4426950408889634
    K = np.zeros((n_seq, hd), np.float32)
    K[0, 0] = K[1, 1] = K[2, 2] = 1.0
    K[3:, 3] = -1.0
    V = np.zeros((n_seq, hd), np.float32)
    V[1], V[2] = 8.0, -8.0
    rng = np.random.default_rng(11)
    a, b = rng.random((2, n_tok, n_head))
    u = 1.0 / (scale * log2e)  # q component giving one log2 unit of score
    q = np.zeros((n_tok, n_head, hd), np.float32)
    q[..., 0] = 20.0 * u
    q[..., 1] = (20.0 - a) * u
    q[..., 2] = (20.0 - b) * u
    q[..., 3] = 40.0 * u
    q = q.reshape(n_tok, n_head * hd)
    Kb, Vb = nh.bf16_round(K), nh.bf16_round(V)
    pos0 = n_seq - n_tok
    kw = dict(n_head=n_head, n_kv=n_kv, head_dim=hd, scale=scale)
    say("case prefill fp16 weights at the copy's limit (V +-8), 256 tokens")
    with nh.KVCache([n_seq], [hd]) as kv:
        kv.append(0, 0, Kb, Vb)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, Kb, Vb, kv_bf16=True, rows=n_seq, pos0=pos0, n_seq=n_seq, **kw)
    # the three weights per row (exact softmax of the exact scores) and the bound
    qs = q.reshape(n_tok, n_head, hd).astype(np.float64)
    s = scale * log2e * qs[..., :3]
    w = np.exp2(s - s.max(axis=-1, keepdims=True))
    w /= w.sum(axis=-1, keepdims=True)
    out = (w * np.array([0.0, 8.0, -8.0])).sum(axis=-1)
    bound = 2.0 ** -11 * (w * np.abs(np.array([0.0, 8.0, -8.0]) - out[..., None])).sum(axis=-1) + 2e-6
    d = np.abs(got.astype(np.float64) - want).reshape(n_tok, n_head, hd).max(axis=-1)
    say(f"  max-abs {d.max():.3e}; largest error / bound {(d / bound).max():.3f}; largest bound {bound.max():.3e}")
    assert np.all(d <= bound)
    assert d.max() <= 5e-3


def test_fp16_shadow_follows_current_contents(monkeypatch):
    """V's fp16 copy counts its elements beyond its limit as they are written
    and replaced: once the ring row holding such a value is overwritten (by a
    raw append or an F32 append), prefill is back on the fp16 path and gives
    the bits of a cache that never held it. A cache still holding one gives the
    bits of the bf16 path (NNC_HIP_F16_SHADOW=0)."""
    cfg = synth.CONFIGS["D"]
    rows, window, n_seq, n_tok = 1024, 512, 2048, 64
    pos0 = n_seq - n_tok
    k, v = synth.kv_rows_f32(cfg, 0, np.arange(n_seq))
    v_bad = v.copy()
    v_bad[100, 9] = 1.0e5  # position 100: row 100, overwritten by position 1124
    q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, n_seq), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    kb, vb, vb_bad = nh.bf16_round(k), nh.bf16_round(v), nh.bf16_round(v_bad)

    def attend(fill, label):
        say(f"case shadow contents: {label}")
        with nh.KVCache([rows], [cfg.kv_dim]) as kv:
            fill(kv)
            return kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)

    clean = attend(lambda kv: kv.append(0, 1024, kb[1024:], vb[1024:]), "positions 1024.. only")

    def raw(kv):
        kv.append(0, 0, kb[:1024], vb_bad[:1024])
        kv.append(0, 1024, kb[1024:], vb[1024:])

    def f32(kv):
        kv.append_f32(0, 0, k[:1024], v_bad[:1024])
        kv.append_f32(0, 1024, k[1024:], v[1024:])

    assert np.array_equal(attend(raw, "raw append, row overwritten").view(np.uint32), clean.view(np.uint32))
    assert np.array_equal(attend(f32, "F32 append, row overwritten").view(np.uint32), clean.view(np.uint32))

    def kept(kv):  # the same value at position 1124 stays in the ring
        kv.append(0, 0, kb[:1024], vb[:1024])
        vb2 = vb.copy()
        vb2[1124, 9] = vb_bad[100, 9]
        kv.append(0, 1024, kb[1024:], vb2[1024:])
        kv.append(0, 1124, kb[1124:1125], vb[1124:1125])  # and is overwritten by the same position again

    assert np.array_equal(attend(kept, "value written, then replaced in place").view(np.uint32), clean.view(np.uint32))

    def held(kv):  # position 1100 (outside the window of every query) keeps it
        vb2 = vb.copy()
        vb2[1100, 9] = vb_bad[100, 9]
        kv.append(0, 1024, kb[1024:], vb2[1024:])

    still = attend(held, "value held outside the window")
    monkeypatch.setenv("NNC_HIP_F16_SHADOW", "0")
    plain = attend(lambda kv: kv.append(0, 1024, kb[1024:], vb[1024:]), "no shadow")
    monkeypatch.delenv("NNC_HIP_F16_SHADOW")
    assert np.array_equal(still.view(np.uint32), plain.view(np.uint32))
    assert not np.array_equal(plain.view(np.uint32), clean.view(np.uint32))


def test_f32_batch_uses_exact_path(orc):
    """F32 K/V batches above 16 tokens run the tiled fp32-MFMA kernel (exact
    fp32 products): the F32 bound holds."""
    cfg = synth.CONFIGS["A"]
    got, want = run_case(orc, cfg, 2, n_seq=1024, pos0=1000, n_tok=24)
    assert errors(got, want)[0] <= 1e-3


# ---- append, fill, errors ---------------------------------------------------------------

def test_append_rounds_like_nnc_and_wraps():
    rng = np.random.default_rng(11)
    rows, kv_dim = 256, 64
    with nh.KVCache([rows], [kv_dim], bf16=True) as kv:
        k = rng.standard_normal((40, kv_dim)).astype(np.float32) * 3
        v = rng.standard_normal((40, kv_dim)).astype(np.float32)
        k[0, :4] = np.array([0x3F808000, 0x3F818000, 0x7F800000, 0x80000000], np.uint32).view(np.float32)
        say("case append_f32 with a wrap at row 256")
        kv.append_f32(0, 230, k, v)  # positions 230..269: rows 230..255 then 0..13
        K, V = kv.read(0, 0, rows)
        idx = np.arange(230, 270) % rows
        assert np.array_equal(K[idx], nh.bf16_round(k)) and np.array_equal(V[idx], nh.bf16_round(v))
        kb, vb = nh.bf16_round(k * 2), nh.bf16_round(v * 2)
        kv.append(0, 250, kb, vb)  # raw BF16 rows, wrapping too
        K, V = kv.read(0, 0, rows)
        idx = np.arange(250, 290) % rows
        assert np.array_equal(K[idx], kb) and np.array_equal(V[idx], vb)
    with nh.KVCache([64], [64], bf16=False) as kv:
        kv.append_f32(0, 3, k[:10], v[:10])
        K, _ = kv.read(0, 3, 10)
        assert np.array_equal(K, k[:10])


def test_device_fill_matches_host_generator():
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    n = 1 << 16
    ptr = C.c_void_p()
    assert hip.hipMalloc(C.byref(ptr), C.c_size_t(n * 4)) == 0
    try:
        out = np.empty(n, dtype=np.float32)
        for norm in (0, 128):
            say(f"case fill_normal norm_dim {norm}")
            nh.fill_normal(ptr.value, n, 777, norm, False)
            assert hip.hipDeviceSynchronize() == 0
            assert hip.hipMemcpy(C.c_void_p(out.ctypes.data), ptr, C.c_size_t(n * 4), 2) == 0
            want = synth.normal(777, n)
            if norm:
                want = synth.rmsnorm_heads(want.reshape(1, -1), norm).reshape(-1)
            assert np.allclose(out, want, rtol=1e-5, atol=1e-5)
    finally:
        hip.hipFree(ptr)


def test_device_errors_map_to_nnc_statuses():
    with nh.KVCache([300], [1024]) as kv:
        cases = [
            (dict(pos0=300, n_seq=301, n_head=32, n_kv=8, head_dim=128), nh.NncStatus.CONTEXT_FULL),
            (dict(pos0=0, n_head=30, n_kv=8, head_dim=128), nh.NncStatus.INVALID_ARGUMENT),
            (dict(pos0=0, n_head=32, n_kv=4, head_dim=128), nh.NncStatus.INVALID_ARGUMENT),
            (dict(pos0=0, n_head=64, n_kv=2, head_dim=512), nh.NncStatus.UNSUPPORTED_MODEL),
            (dict(pos0=-1, n_head=32, n_kv=8, head_dim=128), nh.NncStatus.INVALID_ARGUMENT),
        ]
        for kw, status in cases:
            q = np.zeros((1, kw["n_head"] * kw["head_dim"]), dtype=np.float32)
            with pytest.raises(nh.NncError) as e:
                kv.attend(0, q, scale=0.1, **kw)
            assert e.value.status == status, kw
        q = np.zeros((1, 4096), dtype=np.float32)
        with pytest.raises(nh.NncError) as e:
            kv.attend(1, q, pos0=0, n_head=32, n_kv=8, head_dim=128, scale=0.1)
        assert e.value.status == nh.NncStatus.INVALID_ARGUMENT
        with pytest.raises(nh.NncError):
            kv.append(0, 0, np.zeros((301, 1024), np.uint16), np.zeros((301, 1024), np.uint16))

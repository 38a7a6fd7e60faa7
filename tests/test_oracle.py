"""Pins the CPU oracle (oracle/nnc_oracle.cpp) before any GPU result is
compared with it:

- against the reference's own test of its attention kernels, same recipe and
  tolerance (reference src/appnnc/tests.cpp:2448-2497);
- against closed forms that a dropped term, a wrong index or a swapped
  operand would break;
- against the invariants the reference tests (block split and thread split
  do not change the result, decode equals a batch: reference
  tests.cpp:2631-2661);
- against the reference's compiled kernels (oracle/_ref), where built.
"""
from __future__ import annotations

import numpy as np
import pytest

from libllmcpu_amd import synth


def ref_attention(q, K, V, group, hd, scale):
    """Double-precision softmax attention of `group` heads over every row of
    K/V (the scalar reference of reference tests.cpp:2424-2446), numpy."""
    out = np.zeros((group, hd), dtype=np.float64)
    Kd = K.astype(np.float64)
    Vd = V.astype(np.float64)
    for h in range(group):
        s = Kd @ q[h * hd:(h + 1) * hd].astype(np.float64) * scale
        w = np.exp(s - s.max())
        out[h] = (w @ Vd) / w.sum()
    return out


def bf16_widen(x):
    from libllmcpu_amd import bf16_round, bf16_to_f32

    return bf16_to_f32(bf16_round(x))


# ---- the reference's own kernel test ---------------------------------------------------

@pytest.mark.parametrize("which", [0, 1, 2, 3])
def test_attn_blocks_reference_recipe(orc, which):
    """tests.cpp:2450-2496: group 3, 2 KV heads, 600 keys in blocks of
    100 / 256 / 244 on KV head 1, F32 then BF16 K/V, against the double
    reference at |d| <= 1e-4 (1 + |ref|)."""
    hd, q, K, V = orc.ref_fixture_attn_blocks(which)
    bf16 = which >= 2
    group, n_kv = 3, 2
    kv_stride = n_kv * hd
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    if bf16:
        Kb, Vb = orc.bf16_round(K), orc.bf16_round(V)
        K, V = bf16_widen(K), bf16_widen(V)
        kp, vp = Kb, Vb
    else:
        kp, vp = K, V
    acc = None
    k0 = 0
    for n in (100, 256, 244):
        kb = np.ascontiguousarray(kp.reshape(-1)[k0 * kv_stride + hd:])
        vb = np.ascontiguousarray(vp.reshape(-1)[k0 * kv_stride + hd:])
        part = orc.attn_block(q, kb, vb, bf16, kv_stride, n, hd, group, scale)
        acc = part if acc is None else orc.attn_merge(acc, part, hd, group)
        k0 += n
    out = orc.attn_finish(acc, hd, group)
    want = ref_attention(q, K[:, hd:], V[:, hd:], group, hd, float(scale))
    assert np.all(np.abs(out - want) <= 1e-4 * (1.0 + np.abs(want)))


def test_ref_fixture_matches_reference_kernels(orc, ref):
    """The same case through the reference's compiled nnc_attn_block / merge / finish."""
    for which in range(4):
        hd, q, K, V = orc.ref_fixture_attn_blocks(which)
        bf16 = which >= 2
        kp, vp = (orc.bf16_round(K), orc.bf16_round(V)) if bf16 else (K, V)
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
        outs = []
        for lib in (orc, ref):
            acc = None
            k0 = 0
            for n in (100, 256, 244):
                kb = np.ascontiguousarray(kp.reshape(-1)[k0 * 2 * hd + hd:])
                vb = np.ascontiguousarray(vp.reshape(-1)[k0 * 2 * hd + hd:])
                part = lib.attn_block(q, kb, vb, bf16, 2 * hd, n, hd, 3, scale)
                acc = part if acc is None else lib.attn_merge(acc, part, hd, 3)
                k0 += n
            outs.append(lib.attn_finish(acc, hd, 3))
        assert np.allclose(outs[0], outs[1], rtol=0, atol=2e-6), which


# ---- closed forms ----------------------------------------------------------------------

def _block(orc, q, K, V, hd, group, scale, bf16=False):
    kv = K.shape[1]
    part = orc.attn_block(q, K, V, bf16, kv, K.shape[0], hd, group, scale)
    return orc.attn_finish(part, hd, group), part


def test_closed_form_one_key_gives_its_value(orc):
    rng = np.random.default_rng(1)
    q = rng.standard_normal(2 * 64).astype(np.float32)
    K = rng.standard_normal((1, 64)).astype(np.float32)
    V = rng.standard_normal((1, 64)).astype(np.float32)
    out, part = _block(orc, q, K, V, 64, 2, 0.125)
    assert np.array_equal(out[0], V[0]) and np.array_equal(out[1], V[0])
    assert part[0, 65] == 1.0  # l = exp(0)


def test_closed_form_zero_query_gives_mean_of_values(orc):
    rng = np.random.default_rng(2)
    q = np.zeros(64, dtype=np.float32)
    K = rng.standard_normal((37, 64)).astype(np.float32)
    V = rng.standard_normal((37, 64)).astype(np.float32)
    out, part = _block(orc, q, K, V, 64, 1, 0.125)
    assert np.allclose(out[0], V.mean(axis=0), atol=1e-6)
    assert part[0, 64] == 0.0 and part[0, 65] == 37.0


def test_closed_form_identical_keys_give_mean_of_values(orc):
    rng = np.random.default_rng(3)
    q = rng.standard_normal(128).astype(np.float32)
    K = np.tile(rng.standard_normal((1, 128)).astype(np.float32), (50, 1))
    V = rng.standard_normal((50, 128)).astype(np.float32)
    out, _ = _block(orc, q, K, V, 128, 1, 0.1)
    assert np.allclose(out[0], V.mean(axis=0), atol=1e-6)


def test_closed_form_dominant_key_gives_its_value(orc):
    rng = np.random.default_rng(4)
    hd = 64
    q = np.zeros(hd, dtype=np.float32)
    q[0] = 1.0
    K = rng.standard_normal((20, hd)).astype(np.float32) * 0.01
    K[13, 0] = 1000.0  # score 1000 * scale vs ~0: weight 1 to within exp(-~100)
    V = rng.standard_normal((20, hd)).astype(np.float32)
    out, _ = _block(orc, q, K, V, hd, 1, 0.125)
    assert np.allclose(out[0], V[13], atol=1e-6)


def test_closed_form_zero_sum_finishes_to_zero(orc):
    """l == 0 gives 0, not NaN (reference nn_ops.cpp:492)."""
    acc = np.zeros((2, 66), dtype=np.float32)
    acc[:, :64] = 5.0
    out = orc.attn_finish(acc, 64, 2)
    assert np.all(out == 0.0)


def test_merge_equals_single_block_and_is_split_invariant(orc):
    rng = np.random.default_rng(5)
    hd, group, n = 64, 4, 256
    q = rng.standard_normal(group * hd).astype(np.float32)
    K = rng.standard_normal((n, hd)).astype(np.float32)
    V = rng.standard_normal((n, hd)).astype(np.float32)
    whole, _ = _block(orc, q, K, V, hd, group, 0.125)
    for cut in (1, 17, 128, 255):
        a = orc.attn_block(q, K[:cut].copy(), V[:cut].copy(), False, hd, cut, hd, group, 0.125)
        b = orc.attn_block(q, K[cut:].copy(), V[cut:].copy(), False, hd, n - cut, hd, group, 0.125)
        out = orc.attn_finish(orc.attn_merge(a, b, hd, group), hd, group)
        assert np.allclose(out, whole, atol=2e-6), cut
    # the merge is not symmetric in a way a swapped operand would hide: merging
    # in the wrong order still gives the same softmax, so check m and l too
    a = orc.attn_block(q, K[:100].copy(), V[:100].copy(), False, hd, 100, hd, group, 0.125)
    b = orc.attn_block(q, K[100:].copy(), V[100:].copy(), False, hd, 156, hd, group, 0.125)
    m = orc.attn_merge(a, b, hd, group)
    assert np.array_equal(m[:, hd], np.maximum(a[:, hd], b[:, hd]))


# ---- layer-level: dispatch, spans, rings ----------------------------------------------

def _layer_inputs(cfg, layer, rows, n_seq, pos):
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.asarray(pos), cfg.n_head)
    return q, K, V


@pytest.mark.parametrize("key", ["A", "B", "C", "D", "E"])
def test_layer_matches_textbook(orc, key):
    """Each config's shape at a reduced context, decode and a small batch,
    against the double-precision textbook checker."""
    cfg = synth.CONFIGS[key]
    layer = 0  # sliding for C/E
    n_seq = 900
    rows = cfg.layer_rows(layer, n_seq, 16)
    window = cfg.layer_window(layer)
    kw = dict(kv_bf16=cfg.kv_bf16, rows=rows, window=window, n_head=cfg.n_head, n_kv=cfg.n_kv,
              head_dim=cfg.head_dim, scale=cfg.attn_scale)
    for pos in ([n_seq - 1], list(range(n_seq - 5, n_seq))):
        q, K, V = _layer_inputs(cfg, layer, rows, n_seq, pos)
        got = orc.attend_layer(q, K, V, pos0=pos[0], n_seq=n_seq, **kw)
        want = orc.textbook(q, K, V, pos0=pos[0], n_seq=n_seq, **kw)
        assert np.abs(got - want).max() <= 1e-5, (key, len(pos))


def test_thread_split_and_decode_batch_are_bitwise_equal(orc):
    """nnc's result does not depend on the thread split, and decode of each
    token gives the bits a batch gives it (reference tests.cpp:2631-2661,
    docs/design.md:417-419)."""
    cfg = synth.CONFIGS["D"]
    n_seq = 1100
    q, K, V = _layer_inputs(cfg, 0, n_seq, n_seq, range(n_seq - 3, n_seq))
    kw = dict(kv_bf16=True, rows=n_seq, n_seq=n_seq, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    batch1 = orc.attend_layer(q, K, V, pos0=n_seq - 3, threads=1, **kw)
    batch8 = orc.attend_layer(q, K, V, pos0=n_seq - 3, threads=8, **kw)
    assert np.array_equal(batch1, batch8)
    for t in range(3):
        for threads in (1, 8):  # 8 takes the split-K decode path (span >= 256 KiB)
            one = orc.attend_layer(q[t:t + 1], K, V, pos0=n_seq - 3 + t, threads=threads, **kw)
            assert np.array_equal(one[0], batch1[t]), (t, threads)


def test_ring_equals_full_buffer(orc):
    """A sliding layer's ring gives what a full buffer gives (reference
    tests.cpp:2595-2629): window 40, batch 16 -> 256 rows."""
    cfg = synth.AttnConfig(9, "ring", 4, 2, 64, 1, window=40, swa_period=6)
    rows = orc.kv_rows(1200, 40, 16)
    assert rows == 256 and orc.max_rewind(rows, 40) == 216
    n_seq = 1000
    pos = list(range(n_seq - 16, n_seq))
    q, Kf, Vf = _layer_inputs(cfg, 0, n_seq, n_seq, pos)
    _, Kr, Vr = _layer_inputs(cfg, 0, rows, n_seq, pos)
    kw = dict(kv_bf16=True, n_seq=n_seq, window=40, n_head=4, n_kv=2, head_dim=64, scale=0.125, pos0=pos[0])
    full = orc.attend_layer(q, Kf, Vf, rows=n_seq, **kw)
    ring = orc.attend_layer(q, Kr, Vr, rows=rows, **kw)
    assert np.array_equal(full, ring)


def test_layer_matches_reference_dispatch(orc, ref):
    """The oracle's layer call against the reference's kernels and pool."""
    for key in ("A", "C", "D"):
        cfg = synth.CONFIGS[key]
        n_seq = 1300
        for layer in (0, 5):
            rows = cfg.layer_rows(layer, n_seq, 64)
            window = cfg.layer_window(layer)
            pos = list(range(n_seq - 40, n_seq))
            q, K, V = _layer_inputs(cfg, layer, rows, n_seq, pos)
            kw = dict(kv_bf16=cfg.kv_bf16, rows=rows, n_seq=n_seq, window=window, n_head=cfg.n_head, n_kv=cfg.n_kv,
                      head_dim=cfg.head_dim, scale=cfg.attn_scale)
            for p in (pos[-1:], pos):
                a = orc.attend_layer(q[len(pos) - len(p):], K, V, pos0=p[0], **kw)
                b = ref.attend_layer(q[len(pos) - len(p):], K, V, pos0=p[0], **kw)
                assert np.abs(a - b).max() <= 1e-5 * (1 + np.abs(b).max()), (key, layer, len(p))


# ---- spans, layout, dtype and prep ------------------------------------------------------

SPAN_CASES = [  # reference tests.cpp:1664-1674
    (True, 0, 5, 10, 0, 5), (True, 3, 5, 10, 3, 5), (True, 0, 5, 5, 0, 4), (True, 3, 5, 5, 3, 4),
    (False, 0, 5, 10, 0, 9), (False, 4, 5, 10, 3, 7), (False, 4, 0, 10, 0, 2), (False, 4, 9, 10, 7, 9),
    (False, 512, 300, 1000, 44, 556),
]


@pytest.mark.parametrize("case", SPAN_CASES)
def test_attn_span_known_answers(orc, case):
    from libllmcpu_amd import attn_span

    causal, w, pos, n_seq, first, last = case
    assert orc.attn_span(causal, w, pos, n_seq) == (first, last)
    assert attn_span(causal, w, pos, n_seq) == (first, last)


def test_attn_span_matches_reference(orc, ref):
    from libllmcpu_amd import attn_span

    rng = np.random.default_rng(6)
    for _ in range(2000):
        causal = bool(rng.integers(2))
        w = int(rng.choice([0, 1, 3, 40, 512, 1024]))
        n_seq = int(rng.integers(1, 5000))
        pos = int(rng.integers(0, n_seq + 3))
        want = ref.attn_span(causal, w, pos, n_seq)
        assert orc.attn_span(causal, w, pos, n_seq) == want
        assert attn_span(causal, w, pos, n_seq) == want


def test_kv_sizes_match_published_table(orc):
    """K/V bytes at 4096 context with BF16 (reference README.md:128-133):
    Qwen3-4B 576 MiB, Gemma 3 4B 225 MiB, Llama 3.2 1B 128 MiB, Gemma 3 1B 32.5 MiB."""
    from libllmcpu_amd import kv_rows

    def total(cfg, n_ctx=4096, n_batch=16):
        b = 0
        for li in range(cfg.n_layer):
            w = cfg.layer_window(li)
            rows = kv_rows(n_ctx, w, n_batch) if w else n_ctx
            assert rows == (orc.kv_rows(n_ctx, w, n_batch) if w else n_ctx)
            b += 2 * rows * cfg.kv_dim * 2
        return b / 2 ** 20

    assert total(synth.CONFIGS["D"]) == 576.0
    assert total(synth.CONFIGS["E"]) == 225.0
    assert total(synth.CONFIGS["B"]) == 128.0
    assert total(synth.CONFIGS["C"]) == 32.5


def test_bf16_rounding(orc):
    from libllmcpu_amd import bf16_round, bf16_to_f32

    # ties to even on the bit pattern: 0x3f808000 is halfway between 0x3f80 and 0x3f81
    cases = {0x3F808000: 0x3F80, 0x3F818000: 0x3F82, 0x3F808001: 0x3F81, 0x3F807FFF: 0x3F80, 0x00000000: 0x0000,
             0x80000000: 0x8000, 0x7F800000: 0x7F80, 0xFF800000: 0xFF80, 0x3F800000: 0x3F80}
    x = np.array(list(cases), dtype=np.uint32).view(np.float32)
    want = np.array(list(cases.values()), dtype=np.uint16)
    assert np.array_equal(bf16_round(x), want)
    assert np.array_equal(orc.bf16_round(x), want)
    exact = np.array([0.0, 1.0, -1.0, 2.0, 0.5, -0.5, 1024.0, -2048.0], dtype=np.float32)
    assert np.array_equal(bf16_to_f32(bf16_round(exact)), exact)  # reference tests.cpp:473-479
    rng = np.random.default_rng(0xBF16)
    v = rng.uniform(-3, 3, 100000).astype(np.float32)
    assert np.array_equal(bf16_round(v), orc.bf16_round(v))
    r = bf16_to_f32(bf16_round(v))
    assert np.all(np.abs(r - v) / np.maximum(np.abs(v), 1.0) <= 1.0 / 256)  # half an ulp of 7 bits


def test_bf16_rounding_matches_reference(orc, ref):
    from libllmcpu_amd import bf16_round

    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    assert np.array_equal(bf16_round(x), ref.bf16_round(x))


def test_rope_properties_and_reference_formula(orc):
    rng = np.random.default_rng(0x5051)
    x = rng.uniform(-1, 1, 8 * 64).astype(np.float32)
    assert np.allclose(orc.rope(x, 8, 64, 64, 0.0, 10000.0, 0), x, atol=1e-6)  # pos 0 is the identity
    # NEOX against the scalar formula of reference tests.cpp:1239-1262
    H, D, R, pos, base = 4, 64, 32, 17, 1e6
    x = rng.uniform(-1, 1, H * D).astype(np.float32)
    got = orc.rope(x, H, D, R, float(pos), base, 0)
    want = x.copy().reshape(H, D)
    for h in range(H):
        for i in range(R // 2):
            th = pos * np.float32(base) ** (-np.float32(2 * i) / np.float32(R))
            c, s = np.cos(th), np.sin(th)
            a, b = want[h, i], want[h, i + R // 2]
            want[h, i], want[h, i + R // 2] = c * a - s * b, s * a + c * b
    assert np.allclose(got, want.reshape(-1), rtol=1e-5, atol=1e-5)
    # the package's NORM RoPE (config B's prep) against the oracle's
    x = rng.standard_normal((3, 2 * 64)).astype(np.float32)
    pos = np.array([5, 600, 4095])
    mine = synth.rope(x, pos, 64, 500000.0, "norm")
    for j in range(3):
        assert np.allclose(mine[j], orc.rope(x[j], 2, 64, 64, float(pos[j]), 500000.0, 1), atol=2e-6)
    # rotation keeps each pair's magnitude
    m0 = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
    m1 = mine[:, 0::2] ** 2 + mine[:, 1::2] ** 2
    assert np.allclose(m0, m1, rtol=1e-4)


def test_rope_and_rmsnorm_match_reference(orc, ref):
    rng = np.random.default_rng(8)
    x = rng.standard_normal(8 * 128).astype(np.float32)
    for mode in (0, 1):
        for pos in (0.0, 7.0, 4095.0, 32767.0):
            a = orc.rope(x, 8, 128, 128, pos, 500000.0, mode)
            b = ref.rope(x, 8, 128, 128, pos, 500000.0, mode)
            assert np.array_equal(a, b), (mode, pos)
    a = orc.rmsnorm_groups(x, 128)
    b = ref.rmsnorm_groups(x, 128)
    assert np.array_equal(a, b)
    c = synth.rmsnorm_heads(x.reshape(1, -1), 128).reshape(-1)
    assert np.allclose(c, b, rtol=1e-6, atol=1e-7)
    assert np.allclose(np.sqrt((c.reshape(8, 128) ** 2).mean(axis=1)), 1.0, atol=1e-3)

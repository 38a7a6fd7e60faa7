"""The step before the attention core (reference model.cpp:1616-1691): per-head
RMSNorm of Q/K (gamma) and V (none), RoPE of Q and K, the K/V append.

CPU: the oracle against the reference's own RoPE / RMSNorm outputs
(tests/golden/reference_vectors.npz), its composition against the
reference's pieces called in the reference's order, and closed forms.
GPU: nnc_hip_kv_prep_append_device against the same vectors and against
the oracle over model-shaped cases, then prep + attend end to end.

Tolerances. None for the step itself: q, F32 K/V and BF16 K/V bits equal
the reference's (the oracle is bit for bit against the reference's compiled
RoPE and RMSNorm; the device takes the same sums in the same order and the
rotation angles' cos/sin from the host's libm, as the reference does). End to
end: the attention bound of the BF16 cache, 5e-3."""
from __future__ import annotations

import zlib
from pathlib import Path

import numpy as np
import pytest

import libllmcpu_amd as nh

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def say(msg):
    print(msg, flush=True)


# ---- CPU: the oracle --------------------------------------------------------------------

def test_rope_ff_and_norms_match_reference_vectors(orc, gold):
    x = gold["rope/in"]
    ff = gold["rope_ff/factors"]
    for mode in (0, 1):
        for n_rot in (128, 64):
            for pos in (7, 32767):
                got = orc.rope_ff(x, 4, 128, n_rot, float(pos), 1000000.0, mode, ff[: n_rot // 2])
                assert np.array_equal(got, gold[f"rope_ff/{mode}/{n_rot}/{pos}"]), (mode, n_rot, pos)
    assert np.array_equal(orc.rmsnorm_gamma(x, 128, gold["rmsnorm_gamma/gamma"]), gold["rmsnorm_gamma/out"])
    x80 = gold["rmsnorm_gamma80/in"]
    assert np.array_equal(orc.rmsnorm_gamma(x80, 80, gold["rmsnorm_gamma80/gamma"]), gold["rmsnorm_gamma80/out"])
    assert np.array_equal(orc.rmsnorm_plain(x80, 80), gold["rmsnorm_plain80/out"])


def test_rope_and_norms_bitwise_against_reference(orc, ref):
    """The restatements give the reference's compiled bits over random inputs:
    RoPE in both modes, with and without frequency factors, positions up to
    2^17 and fractional (scaled) positions; RMSNorm with and without gamma at
    head sizes with and without a tail past the last run of eight."""
    rng = np.random.default_rng(21)
    for mode in (0, 1):
        for n_rot, hd in ((64, 64), (64, 128), (128, 128), (256, 256), (32, 80)):
            ff = np.exp(rng.uniform(0.0, 3.0, n_rot // 2)).astype(np.float32)
            for pos in (1.0, 77.0, 4095.0, 32767.0, 131071.0, 1234.5):
                x = (2.0 * rng.standard_normal(4 * hd)).astype(np.float32)
                for f in (None, ff):
                    a = orc.rope_ff(x, 4, hd, n_rot, pos, 1000000.0, mode, f)
                    b = ref.rope_ff(x, 4, hd, n_rot, pos, 1000000.0, mode, f)
                    assert np.array_equal(a, b), (mode, n_rot, hd, pos, f is None)
    for dim in (4, 6, 12, 64, 80, 84, 128, 136, 256, 512):
        x = (2.0 * rng.standard_normal(300 * dim)).astype(np.float32)
        g = rng.uniform(0.5, 1.5, dim).astype(np.float32)
        assert np.array_equal(orc.rmsnorm_gamma(x, dim, g), ref.rmsnorm_gamma(x, dim, g)), dim
        assert np.array_equal(orc.rmsnorm_plain(x, dim), ref.rmsnorm_plain(x, dim)), dim


def test_rope_closed_forms(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(2 * 64).astype(np.float32)
    for mode in (0, 1):
        # position 0 rotates by nothing; n_rot 0 leaves everything
        assert np.array_equal(orc.rope_ff(x, 2, 64, 64, 0.0, 10000.0, mode), x)
        assert np.array_equal(orc.rope_ff(x, 2, 64, 0, 123.0, 10000.0, mode), x)
        # a rotation keeps each pair's length; lanes past n_rot pass through
        y = orc.rope_ff(x, 2, 64, 32, 77.0, 10000.0, mode).reshape(2, 64)
        xr = x.reshape(2, 64)
        pairs = [(i, i + 16) for i in range(16)] if mode == 0 else [(2 * i, 2 * i + 1) for i in range(16)]
        for a, b in pairs:
            assert np.allclose(np.hypot(y[:, a], y[:, b]), np.hypot(xr[:, a], xr[:, b]), rtol=1e-5)
        assert np.array_equal(y[:, 32:], xr[:, 32:])
        # the first pair turns by exactly pos radians (frequency base^0 = 1)
        a, b = pairs[0]
        ang = np.arctan2(y[0, b], y[0, a]) - np.arctan2(xr[0, b], xr[0, a])
        assert abs(np.angle(np.exp(1j * (ang - 77.0)))) < 1e-4
        # a frequency factor of 1e30 switches its pair off
        ff = np.ones(16, np.float32)
        ff[3] = 1e30
        z = orc.rope_ff(x, 2, 64, 32, 77.0, 10000.0, mode, ff).reshape(2, 64)
        a, b = pairs[3]
        assert np.allclose(z[:, [a, b]], xr[:, [a, b]], atol=1e-6)
    # RMSNorm without gamma gives unit RMS; gamma scales each lane
    n = orc.rmsnorm_plain(x, 64).reshape(2, 64)
    assert np.allclose(np.sqrt((n.astype(np.float64) ** 2).mean(axis=1)), 1.0, atol=1e-5)
    g = np.linspace(0.5, 2.0, 64).astype(np.float32)
    assert np.allclose(orc.rmsnorm_gamma(x, 64, g).reshape(2, 64), n * g, rtol=1e-6, atol=1e-7)


def test_prep_append_composes_the_reference_pieces(orc, ref):
    """orc_prep_append against the reference's own RMSNorm, RoPE and BF16
    rounding applied in the order of reference model.cpp:1616-1691."""
    rng = np.random.default_rng(11)
    n_tok, n_head, n_kv, hd, rows, pos0 = 5, 8, 2, 64, 8, 6  # the batch wraps the 8-row buffer
    q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
    qg = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    kg = rng.uniform(0.5, 1.5, hd).astype(np.float32)
    ff = np.exp(rng.uniform(0, 2, hd // 4)).astype(np.float32)
    kw = dict(n_rot=hd // 2, base=10000.0, pos_scale=0.5, mode=0, freq_factors=ff)
    for bf16 in (True, False):
        K0 = np.zeros((rows, n_kv * hd), np.uint16 if bf16 else np.float32)
        qo, Ko, Vo = orc.prep_append(q, k, v, K0, K0.copy(), n_head=n_head, n_kv=n_kv, head_dim=hd, pos0=pos0,
                                     kv_bf16=bf16, q_gamma=qg, k_gamma=kg, v_norm=True, **kw)
        want_q = ref.rmsnorm_gamma(q.reshape(-1), hd, qg).reshape(n_tok, -1)
        want_k = ref.rmsnorm_gamma(k.reshape(-1), hd, kg).reshape(n_tok, -1)
        want_v = ref.rmsnorm_plain(v.reshape(-1), hd).reshape(n_tok, -1)
        for t in range(n_tok):
            rpos = np.float32(pos0 + t) * np.float32(0.5)
            want_q[t] = ref.rope_ff(want_q[t], n_head, hd, hd // 2, float(rpos), 10000.0, 0, ff)
            want_k[t] = ref.rope_ff(want_k[t], n_kv, hd, hd // 2, float(rpos), 10000.0, 0, ff)
        assert np.array_equal(qo, want_q)
        for t in range(n_tok):
            r = (pos0 + t) % rows
            if bf16:
                assert np.array_equal(Ko[r], ref.bf16_round(want_k[t])), t
                assert np.array_equal(Vo[r], ref.bf16_round(want_v[t])), t
            else:
                assert np.array_equal(Ko[r], want_k[t])
                assert np.array_equal(Vo[r], want_v[t])
        untouched = sorted(set(range(rows)) - {(pos0 + t) % rows for t in range(n_tok)})
        assert not Ko[untouched].any() and not Vo[untouched].any()


# ---- GPU: the device step ------------------------------------------------------------------

@pytest.mark.gpu
def test_hip_prep_matches_reference_vectors(gold):
    """The device step against the reference's own RoPE and RMSNorm outputs."""
    x = gold["rope/in"].reshape(1, 4 * 128)
    ff = gold["rope_ff/factors"]
    dummy = np.zeros((1, 128), np.float32)
    with nh.KVCache([8], [128], bf16=False) as kv:
        for mode in (0, 1):
            for n_rot in (128, 64):
                for pos in (7, 32767):
                    say(f"case golden rope mode {mode} n_rot {n_rot} pos {pos}")
                    got = kv.prep_append(0, x, dummy, dummy, pos0=pos, n_head=4, n_kv=1, head_dim=128, n_rot=n_rot,
                                         base=1000000.0, mode=mode, freq_factors=ff[: n_rot // 2])
                    assert np.array_equal(got.reshape(-1), gold[f"rope_ff/{mode}/{n_rot}/{pos}"])
        say("case golden rmsnorm gamma")
        got = kv.prep_append(0, x, dummy, dummy, pos0=0, n_head=4, n_kv=1, head_dim=128,
                             q_gamma=gold["rmsnorm_gamma/gamma"])
        assert np.array_equal(got.reshape(-1), gold["rmsnorm_gamma/out"])
    x80 = gold["rmsnorm_gamma80/in"].reshape(1, 6 * 80)
    with nh.KVCache([4], [480], bf16=False) as kv:
        say("case golden rmsnorm 80 (Q gamma, V plain, F32 cache)")
        got = kv.prep_append(0, x80, x80, x80, pos0=1, n_head=6, n_kv=6, head_dim=80,
                             q_gamma=gold["rmsnorm_gamma80/gamma"], v_norm=True)
        assert np.array_equal(got.reshape(-1), gold["rmsnorm_gamma80/out"])
        K, V = kv.read(0, 1, 1)
        assert np.array_equal(K.reshape(-1), x80.reshape(-1))  # no K norm, no RoPE: stored as given
        assert np.array_equal(V.reshape(-1), gold["rmsnorm_plain80/out"])


PREP_CASES = {
    # name: (n_head, n_kv, hd, n_tok, pos0, rows, bf16, options)
    "llama3_norm_rope": (32, 8, 64, 16, 4000, 4096, True, dict(n_rot=64, base=500000.0, mode=1)),
    "qwen3_qk_norm_neox": (32, 8, 128, 512, 3584, 4096, True, dict(qg=True, kg=True, n_rot=128, base=1000000.0,
                                                                      mode=0)),
    "gemma3_global_scaled": (4, 1, 256, 8, 8000, 8192, True, dict(qg=True, kg=True, n_rot=256, base=1000000.0,
                                                                   mode=0, pos_scale=0.125)),
    "gemma4_partial_ff_vnorm_ring": (8, 4, 256, 12, 250, 256, True, dict(qg=True, kg=True, v_norm=True, n_rot=64,
                                                                          base=10000.0, mode=0, ff=True)),
    "f32_cache_one_token": (16, 4, 128, 1, 32767, 32768, False, dict(kg=True, n_rot=128, base=10000.0, mode=1)),
    # 40 tokens wrapping a 256-row ring: V and its fp16 copy by 32-row groups, partial at both ends
    "ring_wrap_groups": (8, 2, 128, 40, 250, 256, True, dict(qg=True, kg=True, n_rot=128, base=10000.0, mode=0)),
    "no_rope_hd80": (6, 2, 80, 3, 5, 16, True, dict(qg=True, kg=True, n_rot=0)),
    # a head size with a tail past the last run of eight, NORM pairs with factors, far positions in a ring
    "hd100_tail_norm_ff_far": (4, 2, 100, 5, 131000, 256, True, dict(qg=True, kg=True, v_norm=True, n_rot=100,
                                                                     base=1000000.0, mode=1, ff=True)),
}


def _sweep_cases(n: int, seed: int = 31337) -> dict:
    """Seeded shapes beside the named ones: even head sizes up to 512 (with
    tails past the last run of eight), groups 1-8, whole and partial RoPE in
    both pair layouts with and without frequency factors, norms on or off,
    1 to 512 tokens at far positions, plain buffers and wrapping rings, BF16
    and F32 caches."""
    rng = np.random.default_rng(seed)
    out = {}
    for i in range(n):
        hd = int(rng.choice([36, 64, 80, 96, 100, 128, 256, 512]))
        n_kv = int(rng.choice([1, 2, 4, 8]))
        while (n_kv * hd) % 8:  # the cache's rows are whole 16-byte runs
            n_kv *= 2
        group = int(rng.choice([1, 2, 4, 8]))
        n_rot = int(rng.choice([0, hd, 2 * (hd // 4), min(64, hd)]))
        o = dict(qg=bool(rng.random() < 0.7), kg=bool(rng.random() < 0.7), v_norm=bool(rng.random() < 0.3), n_rot=n_rot,
                 base=float(rng.choice([10000.0, 500000.0, 1000000.0])), mode=int(rng.integers(0, 2)),
                 pos_scale=float(rng.choice([1.0, 1.0, 0.25])), ff=bool(n_rot >= 8 and rng.random() < 0.3))
        n_tok = int(rng.choice([1, 3, 16, 17, 100, 512]))
        pos0 = int(rng.choice([0, int(rng.integers(1, 5000)), int(rng.integers(5000, 140000))]))
        if rng.random() < 0.4:
            rows = 256 * int(rng.integers((n_tok + 255) // 256, (n_tok + 255) // 256 + 3))  # a ring
        else:
            pos0 = min(pos0, 9000)
            rows = pos0 + n_tok + int(rng.integers(0, 40))
        out[f"sweep{i:02d}_hd{hd}_g{group}_t{n_tok}"] = (n_kv * group, n_kv, hd, n_tok, pos0, rows,
                                                         bool(rng.random() < 0.75), o)
    return out


SWEEP_CASES = _sweep_cases(16)


def prep_case(name, orc):
    n_head, n_kv, hd, n_tok, pos0, rows, bf16, o = {**PREP_CASES, **SWEEP_CASES}[name]
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    q = (rng.standard_normal((n_tok, n_head * hd)) * 2.0).astype(np.float32)
    k = (rng.standard_normal((n_tok, n_kv * hd)) * 2.0).astype(np.float32)
    v = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
    kw = dict(n_rot=o.get("n_rot", 0), base=o.get("base", 10000.0), pos_scale=o.get("pos_scale", 1.0),
              mode=o.get("mode", 0), v_norm=o.get("v_norm", False), eps=1e-6)
    kw["q_gamma"] = rng.uniform(0.5, 1.5, hd).astype(np.float32) if o.get("qg") else None
    kw["k_gamma"] = rng.uniform(0.5, 1.5, hd).astype(np.float32) if o.get("kg") else None
    if o.get("ff"):
        ff = np.exp(rng.uniform(0.0, 3.0, kw["n_rot"] // 2)).astype(np.float32)
        ff[-4:] = 1e30
        kw["freq_factors"] = ff
    else:
        kw["freq_factors"] = None
    K0 = np.zeros((rows, n_kv * hd), np.uint16 if bf16 else np.float32)
    want_q, want_K, want_V = orc.prep_append(q, k, v, K0, K0.copy(), n_head=n_head, n_kv=n_kv, head_dim=hd, pos0=pos0,
                                             kv_bf16=bf16, **kw)
    return (n_head, n_kv, hd, n_tok, pos0, rows, bf16), q, k, v, kw, (want_q, want_K, want_V)


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(PREP_CASES) + sorted(SWEEP_CASES))
def test_hip_prep_matches_oracle(orc, name):
    (n_head, n_kv, hd, n_tok, pos0, rows, bf16), q, k, v, kw, (want_q, want_K, want_V) = prep_case(name, orc)
    say(f"case prep {name}: {n_tok} tokens at {pos0}, heads {n_head}/{n_kv} x {hd}, rows {rows}, bf16 {bf16}")
    with nh.KVCache([rows], [n_kv * hd], bf16=bf16) as kv:
        got_q = kv.prep_append(0, q, k, v, pos0=pos0, n_head=n_head, n_kv=n_kv, head_dim=hd, **kw)
        K, V = kv.read(0, 0, rows)
    for got, want, what in ((got_q, want_q, "q"), (K, want_K, "K"), (V, want_V, "V")):
        say(f"  {what}: {int((got != want).sum())} of {got.size} elements differ")
        assert np.array_equal(got, want), what


@pytest.mark.gpu
def test_hip_prep_rope_tables_follow_each_call(orc):
    """The bridge keeps the RoPE tables of its last two setups: alternating
    setups (Gemma 3's local and global layers), a repeated call, new positions
    and a third setup that replaces the older table all give the oracle's bits."""
    n_head, n_kv, hd, rows = 4, 2, 128, 64
    rng = np.random.default_rng(31)
    ff = np.exp(rng.uniform(0.0, 2.0, 32)).astype(np.float32)
    setups = {"local": dict(n_rot=128, base=10000.0, pos_scale=1.0, mode=0),
              "global": dict(n_rot=128, base=1000000.0, pos_scale=0.125, mode=0),
              "partial_ff": dict(n_rot=64, base=10000.0, pos_scale=1.0, mode=1, freq_factors=ff)}
    calls = [("local", 100, 3), ("global", 100, 3), ("local", 100, 3), ("global", 103, 1), ("partial_ff", 103, 1),
             ("local", 100, 3), ("partial_ff", 103, 1), ("global", 104, 2)]
    with nh.KVCache([rows], [n_kv * hd], bf16=True) as kv:
        K_host = np.zeros((rows, n_kv * hd), np.uint16)
        V_host = np.zeros_like(K_host)
        for name, pos0, n_tok in calls:
            say(f"case rope table: {name} at {pos0} x {n_tok}")
            q = rng.standard_normal((n_tok, n_head * hd)).astype(np.float32)
            k = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
            v = rng.standard_normal((n_tok, n_kv * hd)).astype(np.float32)
            kw = dict(setups[name], eps=1e-6)
            want_q, K_host, V_host = orc.prep_append(q, k, v, K_host, V_host, n_head=n_head, n_kv=n_kv, head_dim=hd,
                                                     pos0=pos0, kv_bf16=True, **kw)
            got_q = kv.prep_append(0, q, k, v, pos0=pos0, n_head=n_head, n_kv=n_kv, head_dim=hd, **kw)
            K, V = kv.read(0, 0, rows)
            assert np.array_equal(got_q, want_q), (name, pos0)
            assert np.array_equal(K, K_host) and np.array_equal(V, V_host), (name, pos0)


@pytest.mark.gpu
@pytest.mark.parametrize("n_past,n_tok", [(448, 64), (445, 67)])
def test_hip_prep_then_attend_matches_oracle(orc, n_past, n_tok):
    """Prep + attention on the device against the oracle's prep + attention,
    for a Qwen3-shaped batch appended after cached positions: 64 tokens after
    448, and 67 after 445, whose first and last 32-row groups of V's fp16
    copy are shared with rows outside the batch."""
    rng = np.random.default_rng(5)
    n_head, n_kv, hd, rows = 32, 8, 128, 1024
    kw = dict(n_rot=128, base=1000000.0, mode=0, pos_scale=1.0, eps=1e-6,
              q_gamma=rng.uniform(0.5, 1.5, hd).astype(np.float32), k_gamma=rng.uniform(0.5, 1.5, hd).astype(np.float32))
    q = rng.standard_normal((n_past + n_tok, n_head * hd)).astype(np.float32)
    k = rng.standard_normal((n_past + n_tok, n_kv * hd)).astype(np.float32)
    v = rng.standard_normal((n_past + n_tok, n_kv * hd)).astype(np.float32)
    K = np.zeros((rows, n_kv * hd), np.uint16)
    V = K.copy()
    qo, K, V = orc.prep_append(q[:n_past], k[:n_past], v[:n_past], K, V, n_head=n_head, n_kv=n_kv, head_dim=hd, pos0=0,
                               kv_bf16=True, **kw)
    qo, K, V = orc.prep_append(q[n_past:], k[n_past:], v[n_past:], K, V, n_head=n_head, n_kv=n_kv, head_dim=hd,
                               pos0=n_past, kv_bf16=True, **kw)
    scale = 1.0 / np.sqrt(hd)
    want = orc.attend_layer(qo, K, V, kv_bf16=True, rows=rows, pos0=n_past, n_head=n_head, n_kv=n_kv, head_dim=hd,
                            scale=scale)
    say(f"case prep + attend: {n_past} cached + {n_tok} new tokens, qwen3 shape")
    with nh.KVCache([rows], [n_kv * hd], bf16=True) as kv:
        kv.prep_append(0, q[:n_past], k[:n_past], v[:n_past], pos0=0, n_head=n_head, n_kv=n_kv, head_dim=hd, **kw)
        qg = kv.prep_append(0, q[n_past:], k[n_past:], v[n_past:], pos0=n_past, n_head=n_head, n_kv=n_kv, head_dim=hd,
                            **kw)
        got = kv.attend(0, qg, pos0=n_past, n_head=n_head, n_kv=n_kv, head_dim=hd, scale=scale)
    err = float(np.abs(got - want).max())
    say(f"  max-abs {err:.3e}")
    assert err <= 5e-3


@pytest.mark.gpu
def test_hip_prep_refuses_bad_arguments():
    with nh.KVCache([16], [128], bf16=True) as kv:
        for kwargs in [
            dict(n_head=2, n_kv=1, head_dim=128, n_rot=3),  # odd n_rot
            dict(n_head=2, n_kv=1, head_dim=128, n_rot=256),  # n_rot above head_dim
            dict(n_head=2, n_kv=1, head_dim=128, n_rot=128, mode=2),  # no such RoPE mode
            dict(n_head=4, n_kv=2, head_dim=64, n_rot=64, base=0.0),  # no frequency base
            dict(n_head=2, n_kv=2, head_dim=128),  # kv_dim 256, buffer 128
        ]:
            q = np.zeros((1, kwargs["n_head"] * kwargs["head_dim"]), np.float32)
            k = np.zeros((1, kwargs["n_kv"] * kwargs["head_dim"]), np.float32)
            with pytest.raises(nh.NncError) as e:
                kv.prep_append(0, q, k, k, pos0=0, **kwargs)
            assert e.value.status == nh.NncStatus.INVALID_ARGUMENT, kwargs

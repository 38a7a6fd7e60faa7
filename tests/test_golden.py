"""The oracle against the reference's own outputs stored in
tests/golden/reference_vectors.npz (written by tests/golden/make_golden.py
from the reference's libnnc sources compiled in oracle/_ref), and the HIP op
against the same vectors on the GPU.

Inputs are regenerated from the synthetic streams; their SHA-256 must match
the one stored with each vector."""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def sha(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_names(gold):
    return sorted({k.split("/")[1] for k in gold.files if k.startswith("layer/")})


def layer_case(gold, name):
    key = str(gold[f"layer/{name}/config"])
    layer, n_seq, pos0, n_tok, n_batch = (int(v) for v in gold[f"layer/{name}/case"])
    cfg = synth.CONFIGS[key]
    rows = cfg.layer_rows(layer, n_seq, n_batch)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    assert sha(q, K, V) == str(gold[f"layer/{name}/sha256"]), f"{name}: regenerated inputs differ"
    kw = dict(rows=rows, pos0=pos0, n_seq=n_seq, window=cfg.layer_window(layer), causal=True, n_head=cfg.n_head,
              n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    return cfg, q, K, V, kw, gold[f"layer/{name}/out"]


def stored_rows(gold, name, out):
    """The rows of `out` the file holds: every stride-th token."""
    return out[::int(gold[f"layer/{name}/stride"])]


def test_golden_file_holds_every_case(gold):
    """Decode tokens, 8-token batches, and two 64-token chunks (hd 128, and
    hd 256 on a global layer) long enough for the MFMA prefill kernel."""
    assert len(layer_names(gold)) == 9
    for name in ("D_prefill_chunk64", "E_global_chunk64"):
        assert int(gold[f"layer/{name}/case"][3]) >= 64
        assert gold[f"layer/{name}/out"].shape[0] == 16
    assert {f"blocks/{w}/out" for w in range(4)} <= set(gold.files)


def test_oracle_layers_match_reference_vectors(orc, gold):
    """nnc's attention core (decode, prefill chunks, a wrapped ring, F32 and
    BF16) from the oracle against the reference's compiled code: the two
    differ only in exp's polynomial and summation order."""
    for name in layer_names(gold):
        cfg, q, K, V, kw, want = layer_case(gold, name)
        got = stored_rows(gold, name, orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, **kw))
        assert np.all(np.abs(got - want) <= 1e-5 * (1.0 + np.abs(want))), name


def test_oracle_blocks_match_reference_vectors(orc, gold):
    """reference tests.cpp:2450-2496's block case through attn_block / merge / finish."""
    for which in range(4):
        hd, q, K, V = orc.ref_fixture_attn_blocks(which)
        bf16 = which >= 2
        kp, vp = (orc.bf16_round(K), orc.bf16_round(V)) if bf16 else (K, V)
        assert sha(q, kp, vp) == str(gold[f"blocks/{which}/sha256"])
        scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
        acc, k0 = None, 0
        for n in (100, 256, 244):
            kb = np.ascontiguousarray(kp.reshape(-1)[k0 * 2 * hd + hd:])
            vb = np.ascontiguousarray(vp.reshape(-1)[k0 * 2 * hd + hd:])
            part = orc.attn_block(q, kb, vb, bf16, 2 * hd, n, hd, 3, scale)
            acc = part if acc is None else orc.attn_merge(acc, part, hd, 3)
            k0 += n
        got = orc.attn_finish(acc, hd, 3)
        assert np.allclose(got, gold[f"blocks/{which}/out"], rtol=0, atol=2e-6), which


def test_spans_match_reference_vectors(orc, gold):
    for (c, w, p, n), want in zip(gold["span/args"], gold["span/out"]):
        args = (bool(c), int(w), int(p), int(n))
        assert orc.attn_span(*args) == tuple(want)
        assert nh.attn_span(*args) == tuple(want)


def test_bf16_rounding_matches_reference_vectors(orc, gold):
    x = gold["bf16/in"]
    assert np.array_equal(orc.bf16_round(x), gold["bf16/out"])
    assert np.array_equal(nh.bf16_round(x), gold["bf16/out"])


def test_rope_and_rmsnorm_match_reference_vectors(orc, gold):
    x = gold["rope/in"]
    for mode in (0, 1):
        for pos in (7, 4095):
            got = orc.rope(x, 4, 128, 128, float(pos), 500000.0, mode)
            assert np.allclose(got, gold[f"rope/{mode}/{pos}"], atol=1e-5), (mode, pos)
    # the package's NORM RoPE (config B's prep) is the oracle's mode 1
    mine = synth.rope(x.reshape(1, -1), np.array([4095]), 128, 500000.0, "norm").reshape(-1)
    assert np.allclose(mine, gold["rope/1/4095"], atol=1e-5)
    assert np.allclose(orc.rmsnorm_groups(x, 128), gold["rmsnorm/out"], rtol=1e-6, atol=1e-7)
    assert np.allclose(synth.rmsnorm_heads(x.reshape(1, -1), 128).reshape(-1), gold["rmsnorm/out"], rtol=1e-6,
                       atol=1e-7)


@pytest.mark.gpu
def test_hip_op_matches_reference_vectors(gold):
    """The HIP op through the C ABI against the reference's outputs (bounds:
    1e-3 for F32 K/V, 5e-3 for BF16): decode and 8-token batches through the
    split-K kernels, the 64-token chunks through the MFMA prefill kernel."""
    for name in layer_names(gold):
        cfg, q, K, V, kw, want = layer_case(gold, name)
        print(f"case golden {name}: tokens {kw['pos0']}+{q.shape[0]} rows {kw['rows']}", flush=True)
        with nh.KVCache([kw["rows"]], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
            kv.append(0, 0, K, V)
            got = stored_rows(gold, name, kv.attend(0, q, **{k: v for k, v in kw.items() if k != "rows"}))
        err = float(np.abs(got.astype(np.float64) - want).max())
        print(f"  max-abs {err:.3e}", flush=True)
        assert err <= cfg.tol, (name, err)

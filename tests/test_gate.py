"""Qwen3.5's attention output gate: out *= sigmoid(gate) after the attention
core (reference src/libnnc/model.cpp:1759-1760, nn_ops.cpp:1731-1742).

CPU: the oracle's restatement against the reference's vectors, the
reference's compiled code where it is built, and the closed forms
(sigmoid(0) = 1/2, the saturated ends, sigmoid(g) + sigmoid(-g) = 1).
GPU: the gated entry points against the oracle (attention, then the gate),
for decode, a session batch (bit-identical to its one-token calls), a
prefill batch and F32 K/V; max-abs bounds 5e-3 (BF16 K/V) and 1e-3 (F32)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from libllmcpu_amd import synth

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def test_gate_matches_reference_vectors(orc, gold):
    got = orc.mul_sigmoid(gold["gate/y"], gold["gate/g"])
    assert np.allclose(got, gold["gate/out"], rtol=1e-6, atol=1e-30)


def test_gate_matches_reference_code(orc, ref):
    rng = np.random.default_rng(5)
    for n in (1, 7, 8, 9, 4096 + 5):
        y = rng.standard_normal(n).astype(np.float32)
        g = (rng.standard_normal(n) * 10).astype(np.float32)
        assert np.allclose(orc.mul_sigmoid(y, g), ref.mul_sigmoid(y, g), rtol=1e-6, atol=1e-30), n


def test_gate_closed_forms(orc):
    y = np.linspace(-3, 3, 17, dtype=np.float32)
    assert np.array_equal(orc.mul_sigmoid(y, np.zeros_like(y)), y * np.float32(0.5))
    assert np.array_equal(orc.mul_sigmoid(y, np.full_like(y, 100.0)), y)
    assert np.all(orc.mul_sigmoid(y, np.full_like(y, -200.0)) == 0.0)
    g = np.random.default_rng(1).standard_normal(17).astype(np.float32) * 4
    assert np.allclose(orc.mul_sigmoid(y, g) + orc.mul_sigmoid(y, -g), y, atol=1e-6)


def _gated_case(orc, cfg, layer, pos0, n, nh):
    n_seq = pos0 + n
    rows = cfg.layer_rows(layer, n_seq, 16)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, n_seq), cfg.n_head)
    gate = (np.random.default_rng(pos0 + n).standard_normal(q.shape) * 3).astype(np.float32)
    kw = dict(window=cfg.layer_window(layer), causal=True, n_head=cfg.n_head, n_kv=cfg.n_kv,
              head_dim=cfg.head_dim, scale=cfg.attn_scale)
    print(f"case gated {cfg.name} layer {layer}: tokens {pos0}+{n}", flush=True)
    with nh.KVCache([rows], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, gate=gate, **kw)
        single = None
        if 1 < n <= 16:
            single = np.stack([kv.attend(0, q[t:t + 1], pos0=pos0 + t, n_seq=pos0 + t + 1, gate=gate[t:t + 1],
                                         **kw)[0] for t in range(n)])
    want = orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.mul_sigmoid(want, gate).reshape(got.shape)
    return got, want, single


@pytest.mark.gpu
@pytest.mark.parametrize("key,layer,pos0,n", [
    ("D", 0, 4095, 1),     # decode, Qwen3 head shape
    ("D", 1, 2000, 16),    # a session batch
    ("D", 2, 448, 64),     # the prefill kernel
    ("A", 0, 1000, 3),     # F32 K/V
    ("C", 0, 3000, 1),     # local layer in a ring, hd 256
])
def test_gated_attention_matches_oracle(orc, key, layer, pos0, n):
    import libllmcpu_amd as nh

    cfg = synth.CONFIGS[key]
    got, want, single = _gated_case(orc, cfg, layer, pos0, n, nh)
    err = float(np.abs(got.astype(np.float64) - want).max())
    print(f"  max-abs {err:.3e}", flush=True)
    assert err <= cfg.tol
    if single is not None:
        assert np.array_equal(got.view(np.uint32), single.view(np.uint32))

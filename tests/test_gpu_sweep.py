"""A seeded sweep of random attention calls against the oracle: head_dim
(the MFMA sizes, the tiled kernel's multiples of 16, and 36), query groups 1
to 8 (and 3), BF16 and F32 caches, causal spans over full buffers and over
rings with sliding windows, bidirectional whole-input batches, and batch
sizes from one token (decode) through a session batch (16) to chunks of
more than 16 tokens (prefill, tiled and split-K kernels). Each case is drawn
from its own seed, prints its parameters before its GPU call, and must stay
within the F32 (1e-3) or BF16 (5e-3) bound of the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, say

pytestmark = pytest.mark.gpu

HEAD_DIMS = (64, 128, 256, 80, 96, 512, 36)
GROUPS = (1, 2, 3, 4, 8)
N_TOKS = (1, 3, 16, 17, 40, 130)


def draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    hd = int(rng.choice(HEAD_DIMS))
    g = int(rng.choice([x for x in GROUPS if x * hd <= 8192]))
    n_kv = int(rng.choice((1, 2, 4))) if hd <= 256 else 1
    if (n_kv * hd) % 8:  # a cache row is a multiple of 8 elements
        n_kv = 2
    bf16 = bool(rng.random() < 0.7)
    n_tok = int(rng.choice(N_TOKS))
    kind = rng.choice(("causal", "causal", "window", "bidir"))
    if kind == "bidir":
        window = int(rng.choice((0, 128, 300)))
        n_seq = max(n_tok, 2)
        pos0, rows, causal = 0, n_seq, False
        n_tok = n_seq
    else:
        window = int(rng.choice((64, 300, 512))) if kind == "window" else 0
        n_seq = int(rng.integers(n_tok, 2500))
        pos0 = n_seq - n_tok
        rows = nh.kv_rows(n_seq, window, 256) if window else n_seq
        causal = True
    return dict(hd=hd, g=g, n_kv=n_kv, bf16=bf16, n_tok=n_tok, window=window, n_seq=n_seq, pos0=pos0, rows=rows,
                causal=causal)


@pytest.mark.parametrize("seed", range(40))
def test_random_call(orc, seed):
    c = draw(seed)
    cfg = synth.AttnConfig(20 + seed, f"sweep {seed}", c["g"] * c["n_kv"], c["n_kv"], c["hd"], 1, kv_bf16=c["bf16"])
    K, V = synth.cache_buffer(cfg, 0, c["rows"], c["n_seq"])
    q = synth.qk_rows(cfg, 0, 0, np.arange(c["pos0"], c["pos0"] + c["n_tok"]), cfg.n_head)
    kw = dict(window=c["window"], causal=c["causal"], n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    say(f"case sweep {seed}: {c}")
    with nh.KVCache([c["rows"]], [cfg.kv_dim], bf16=c["bf16"]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=c["pos0"], n_seq=c["n_seq"], **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=c["bf16"], rows=c["rows"], pos0=c["pos0"], n_seq=c["n_seq"], **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e}")
    assert ea <= (5e-3 if c["bf16"] else 1e-3)

"""Head shapes outside the MFMA kernels' (head_dim 64/128/256 with groups of
1, 2, 4 or 8) through the generic split-K kernels: nnc runs any even
head_dim up to 512 (reference src/libnnc/model.cpp:714, nn_ops.cpp:1841),
e.g. Gemma 4's global layers at 512, and its own block test uses 36 with a
group of 3 (src/appnnc/tests.cpp:2450-2497). Each shape: decode, a 16-token
session batch whose every token must equal its one-token call bit for bit, a
100-token batch, against the oracle within the BF16 / F32 bound; a windowed
ring; and the shapes the bridge refuses."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import synth

from gpu_util import errors, say

pytestmark = pytest.mark.gpu

SHAPES = (  # (head_dim, n_head, n_kv, BF16)
    (80, 32, 8, True),
    (512, 16, 2, True),
    (36, 6, 2, True),
    (96, 12, 4, False),
    (128, 12, 4, True),  # an MFMA head size with a group of 3
)


@pytest.mark.parametrize("hd,n_head,n_kv,bf16", SHAPES)
def test_generic_head_shapes(orc, hd, n_head, n_kv, bf16):
    cfg = synth.AttnConfig(10, f"hd{hd}", n_head, n_kv, hd, 1, kv_bf16=bf16)
    tol = 5e-3 if bf16 else 1e-3
    n_seq = 3000
    K, V = synth.cache_buffer(cfg, 0, n_seq, n_seq)
    kw = dict(n_head=n_head, n_kv=n_kv, head_dim=hd, scale=cfg.attn_scale)
    with nh.KVCache([n_seq], [cfg.kv_dim], bf16=bf16) as kv:
        kv.append(0, 0, K, V)
        outs = {}
        for pos0, n_tok in ((2999, 1), (2984, 16), (2900, 100)):
            say(f"case head_dim {hd}, {n_head}/{n_kv} heads, {'BF16' if bf16 else 'F32'}: tokens {pos0}+{n_tok}")
            q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, pos0 + n_tok), n_head)
            got = kv.attend(0, q, pos0=pos0, n_seq=pos0 + n_tok, **kw)
            want = orc.attend_layer(q, K, V, kv_bf16=bf16, rows=n_seq, pos0=pos0, n_seq=pos0 + n_tok, **kw)
            ea, er = errors(got, want)
            say(f"  max-abs {ea:.3e} max-rel {er:.3e}")
            assert ea <= tol, (pos0, n_tok)
            outs[(pos0, n_tok)] = (q, got)
        # the session batch: every token gets its one-token call's bits
        q16, got16 = outs[(2984, 16)]
        for t in (0, 7, 15):
            one = kv.attend(0, q16[t:t + 1], pos0=2984 + t, n_seq=2984 + t + 1, **kw)
            assert np.array_equal(one.view(np.uint32), got16[t:t + 1].view(np.uint32)), t


def test_generic_head_shape_windowed_ring(orc):
    """head_dim 80 on a sliding layer: a 768-row ring, window 256, the batch's
    keys wrapping the ring."""
    cfg = synth.AttnConfig(11, "hd80 ring", 16, 4, 80, 1)
    rows, window, n_seq, n_tok = 768, 256, 2000, 40
    K, V = synth.cache_buffer(cfg, 0, rows, n_seq)
    q = synth.qk_rows(cfg, 0, 0, np.arange(n_seq - n_tok, n_seq), cfg.n_head)
    kw = dict(window=window, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=80, scale=cfg.attn_scale)
    say("case head_dim 80 ring, window 256, 40 tokens")
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=n_seq - n_tok, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=n_seq - n_tok, n_seq=n_seq, **kw)
    ea, er = errors(got, want)
    say(f"  max-abs {ea:.3e}")
    assert ea <= 5e-3


@pytest.mark.parametrize("hd,n_head,n_kv", ((129, 8, 8), (514, 4, 4), (64, 17, 1), (384, 48, 2)))
def test_unsupported_head_shapes_are_refused(hd, n_head, n_kv):
    """An odd head_dim, one past 512 and groups above 16 give
    NNC_ERR_UNSUPPORTED_MODEL before any device work."""
    say(f"case refused shape: head_dim {hd}, {n_head}/{n_kv} heads")
    with nh.KVCache([64], [n_kv * hd]) as kv:
        q = np.zeros((1, n_head * hd), np.float32)
        with pytest.raises(nh.NncError) as e:
            kv.attend(0, q, pos0=10, n_head=n_head, n_kv=n_kv, head_dim=hd, scale=0.1)
        assert e.value.status == nh.NncStatus.UNSUPPORTED_MODEL

"""nnc_hip_attend_device_noalloc through the C ABI: the decode kernels'
partials in the library's fixed per-device array instead of the cache's
scratch. Each call must give exactly the bits nnc_hip_attend_device gives for
the same inputs (the same kernels run), on consecutive calls of shrinking
size (the array keeps the previous call's contents), and within the BF16
bound of the oracle; a call whose partials do not fit the array is refused.
Each case prints its name before its GPU calls."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import hip_rt, synth

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)


def test_noalloc_matches_attend_device_on_consecutive_calls(orc):
    cfg = synth.CONFIGS["D"]  # Qwen3-4B: 32 query heads, 8 KV heads, head_dim 128
    rows = 8192
    K, V = synth.cache_buffer(cfg, 0, rows, rows)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    width = cfg.n_head * cfg.head_dim
    with nh.KVCache([rows], [cfg.kv_dim]) as kv:
        kv.append(0, 0, K, V)
        q_dev = hip_rt.malloc(16 * width * 4)
        o_ref = hip_rt.malloc(16 * width * 4)
        o_new = hip_rt.malloc(16 * width * 4)
        try:
            # decode at 8192 keys, a 16-token session batch, then smaller calls
            for pos0, n_tok in ((8191, 1), (8176, 16), (3000, 5), (700, 1)):
                say(f"case noalloc D: tokens {pos0}+{n_tok}")
                q = synth.qk_rows(cfg, 0, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
                hip_rt.to_device(q_dev, q)
                kv.attend_device(0, q_dev, o_ref, n_tok=n_tok, pos0=pos0, **kw)
                kv.attend_device_noalloc(0, q_dev, o_new, n_tok=n_tok, pos0=pos0, **kw)
                kv.sync()
                ref = hip_rt.to_host(np.empty((n_tok, width), np.float32), o_ref)
                got = hip_rt.to_host(np.empty((n_tok, width), np.float32), o_new)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (pos0, n_tok)
                want = orc.attend_layer(q, K, V, kv_bf16=True, rows=rows, pos0=pos0, n_seq=pos0 + n_tok, **kw)
                err = float(np.abs(got.astype(np.float64) - want).max())
                say(f"  bit-identical to attend_device; max-abs vs oracle {err:.3e}")
                assert err <= cfg.tol
        finally:
            for d in (q_dev, o_ref, o_new):
                hip_rt.free(d)


def test_noalloc_refuses_partials_past_the_array():
    # 64 query heads over 8 KV heads, head_dim 256: a 16-token batch at 16k
    # keys leaves about 16 x 64 splits x 8 heads x 8 x 260 floats of partials,
    # far past the 32 MiB array.
    n_head, n_kv, hd, rows = 64, 8, 256, 16384
    with nh.KVCache([rows], [n_kv * hd]) as kv:
        q_dev = hip_rt.malloc(16 * n_head * hd * 4)
        o_dev = hip_rt.malloc(16 * n_head * hd * 4)
        try:
            say("case noalloc oversize batch")
            with pytest.raises(nh.NncError) as e:
                kv.attend_device_noalloc(0, q_dev, o_dev, n_tok=16, pos0=rows - 16, n_head=n_head, n_kv=n_kv,
                                         head_dim=hd, scale=1 / 16)
            assert e.value.status == nh.NncStatus.INVALID_ARGUMENT
            assert "fixed scratch" in e.value.message
            kv.sync()
        finally:
            hip_rt.free(q_dev)
            hip_rt.free(o_dev)

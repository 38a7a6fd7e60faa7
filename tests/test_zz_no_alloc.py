"""nnc_hip_attend_device_noalloc through the C ABI: the decode kernels'
partials in the library's fixed per-device array instead of the cache's
scratch. Each call must give exactly the bits nnc_hip_attend_device gives for
the same inputs (the same kernels run), on consecutive calls of shrinking
size (the array keeps the previous call's contents), and within the BF16
bound of the oracle. The first call on a fresh cache runs under thread-local
HIP graph capture, where any device allocation or synchronisation fails the
capture, and its graph's replays match. A call whose partials do not fit the
array is refused before anything is enqueued. Each case prints its name
before its GPU calls."""
from __future__ import annotations

import numpy as np
import pytest

import libllmcpu_amd as nh
from libllmcpu_amd import hip_rt, synth

pytestmark = pytest.mark.gpu


def say(msg: str) -> None:
    print(msg, flush=True)


def test_noalloc_first_call_is_captured_and_replays(orc):
    """Fresh caches A and B with the same rows: A's first no-alloc calls (a
    decode token, a 16-token session batch and a short-span decode token,
    whose merge runs inside the split launch) are captured into a HIP graph
    (thread-local capture mode: a hipMalloc, hipFree or stream
    synchronisation inside the call would fail hipStreamEndCapture). B runs
    the same calls eagerly through nnc_hip_attend_device. Three replays, each
    after an eager no-alloc call of another size that rewrites the shared
    array, give B's bits."""
    cfg = synth.CONFIGS["D"]  # Qwen3-4B: 32 query heads, 8 KV heads, head_dim 128
    rows = 8192
    K, V = synth.cache_buffer(cfg, 0, rows, rows)
    kw = dict(n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    width = cfg.n_head * cfg.head_dim
    calls = ((8191, 1, 0), (8176, 16, 1), (700, 1, 17))  # (pos0, n_tok, first token slot)
    q = np.concatenate([synth.qk_rows(cfg, 0, 0, np.arange(p, p + n), cfg.n_head) for p, n, _ in calls])
    with nh.KVCache([rows], [cfg.kv_dim]) as kv_a, nh.KVCache([rows], [cfg.kv_dim]) as kv_b:
        kv_a.append(0, 0, K, V)
        kv_b.append(0, 0, K, V)
        kv_a.sync()
        kv_b.sync()
        q_dev = hip_rt.malloc(q.nbytes)
        o_graph = hip_rt.malloc(q.nbytes)
        o_ref = hip_rt.malloc(q.nbytes)
        o_other = hip_rt.malloc(5 * width * 4)
        graph = None
        try:
            hip_rt.to_device(q_dev, q)

            def issue(kv, fn, out):
                for pos0, n_tok, slot in calls:
                    fn(kv, 0, q_dev + 4 * slot * width, out + 4 * slot * width, n_tok=n_tok, pos0=pos0, **kw)

            say("case noalloc D: first calls of a fresh cache under graph capture")
            graph = hip_rt.Graph(kv_a.stream, lambda: issue(kv_a, nh.KVCache.attend_device_noalloc, o_graph))
            say("case noalloc D: the same calls eagerly through attend_device on a second cache")
            issue(kv_b, nh.KVCache.attend_device, o_ref)
            kv_b.sync()
            ref = hip_rt.to_host(np.empty_like(q), o_ref)
            want = np.concatenate([orc.attend_layer(q[s:s + n], K, V, kv_bf16=True, rows=rows, pos0=p, n_seq=p + n, **kw)
                                   for p, n, s in calls])
            err = float(np.abs(ref.astype(np.float64) - want).max())
            say(f"  attend_device max-abs vs oracle {err:.3e}")
            assert err <= cfg.tol
            for rep in range(3):
                say(f"case noalloc D: eager 5-token call, then replay {rep}")
                kv_a.attend_device_noalloc(0, q_dev, o_other, n_tok=5, pos0=3000 + 7 * rep, **kw)
                kv_a.sync()
                hip_rt.to_device(o_graph, np.full_like(q, np.nan))
                graph.launch(kv_a.stream)
                kv_a.sync()
                got = hip_rt.to_host(np.empty_like(q), o_graph)
                assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), rep
        finally:
            if graph is not None:
                graph.close()
            for d in (q_dev, o_graph, o_ref, o_other):
                hip_rt.free(d)


def test_noalloc_matches_attend_device_on_consecutive_calls(orc):
    cfg = synth.CONFIGS["D"]
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
                kv.attend_device_noalloc(0, q_dev, o_new, n_tok=n_tok, pos0=pos0, **kw)
                kv.attend_device(0, q_dev, o_ref, n_tok=n_tok, pos0=pos0, **kw)
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


def test_noalloc_refuses_partials_past_the_array_and_changes_nothing():
    """64 query heads over 8 KV heads, head_dim 256 (every token's own split
    grid: about 64 splits of 8 x 260 floats per KV head). A 16-token batch
    from position 12287: on a 256-CU part the first token (span 12288) runs
    on 192-key splits and the other 15 (spans from 12289) on 256-key splits,
    so the first launch's partials (about 4 MiB) fit the 32 MiB array and the
    second's (about 49 MiB) do not. The call is refused before any launch is
    enqueued: the output keeps its sentinel bits."""
    n_head, n_kv, hd, rows = 64, 8, 256, 16384
    n_tok, pos0 = 16, 12287
    width = n_head * hd
    with nh.KVCache([rows], [n_kv * hd]) as kv:
        q_dev = hip_rt.malloc(n_tok * width * 4)
        o_dev = hip_rt.malloc(n_tok * width * 4)
        try:
            hip_rt.to_device(q_dev, np.ones((n_tok, width), np.float32))
            sentinel = np.full((n_tok, width), 0x7FC01234, np.uint32)
            hip_rt.to_device(o_dev, sentinel)
            say("case noalloc oversize batch (second launch past the array)")
            with pytest.raises(nh.NncError) as e:
                kv.attend_device_noalloc(0, q_dev, o_dev, n_tok=n_tok, pos0=pos0, n_head=n_head, n_kv=n_kv,
                                         head_dim=hd, scale=1 / 16)
            assert e.value.status == nh.NncStatus.INVALID_ARGUMENT
            assert "fixed scratch" in e.value.message
            kv.sync()
            after = hip_rt.to_host(np.empty((n_tok, width), np.uint32), o_dev)
            assert np.array_equal(after, sentinel)
        finally:
            hip_rt.free(q_dev)
            hip_rt.free(o_dev)

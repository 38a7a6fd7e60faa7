"""Helpers shared by the GPU parity tests: a case runner that fills one
layer's cache as a session would have and runs the HIP op and the oracle on
the same inputs."""
from __future__ import annotations

import numpy as np

import libllmcpu_amd as nh
from libllmcpu_amd import synth


def say(msg: str) -> None:
    print(msg, flush=True)


def errors(got, want):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    rel = d / np.maximum(np.abs(want), 1e-6)
    return float(d.max()), float(rel.max())


def run_case(orc, cfg, layer, *, n_seq, pos0, n_tok, n_batch=16, rows=None, threads=8, causal=True):
    """Fills one layer's cache as a session would have (positions 0..n_seq-1),
    runs the op for tokens pos0 .. pos0 + n_tok - 1 on the GPU and on the oracle."""
    window = cfg.layer_window(layer)
    if rows is None:
        rows = cfg.layer_rows(layer, n_seq, n_batch)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    kw = dict(window=window, causal=causal, n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim,
              scale=cfg.attn_scale)
    say(f"case {cfg.name} layer {layer}: n_seq {n_seq} rows {rows} window {window} tokens {pos0}+{n_tok}")
    with nh.KVCache([rows], [cfg.kv_dim], bf16=cfg.kv_bf16) as kv:
        kv.append(0, 0, K, V)
        got = kv.attend(0, q, pos0=pos0, n_seq=n_seq, **kw)
    want = orc.attend_layer(q, K, V, kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, threads=threads, **kw)
    return got, want

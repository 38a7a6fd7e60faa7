"""TEST INFRASTRUCTURE — ctypes bindings of the CPU oracle.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or, in the bench, as the timed CPU
baseline): the product path never calls it.

- ``Oracle`` binds liboracle.so, this repository's restatement of nnc's
  attention core (nnc_oracle.cpp; each function cites the reference lines it
  follows) plus the double-precision textbook checker.
- ``Reference`` binds _ref/libnnc_ref.so: the reference's own libnnc sources,
  compiled from /root/reference by oracle/Makefile, behind a small C driver
  (ref_driver.cpp). It exists only where it was built; it travels to the GPU
  box as a built file.

Build both with ``make -C oracle`` (``build()`` below).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_SO = HERE / "liboracle.so"
REF_SO = HERE / "_ref" / "libnnc_ref.so"
REF_SRC = Path("/root/reference/src/libnnc")

_P = C.c_void_p
_SZ = C.c_size_t
_I = C.c_int
_F = C.c_float


def build(verbose: bool = False) -> None:
    """make -B -C oracle: rebuilds liboracle.so, and _ref/libnnc_ref.so when
    the reference sources are present."""
    r = subprocess.run(["make", "-B", "-C", str(HERE), "-j8"], capture_output=True, text=True)
    if verbose:
        print(r.stdout)
    if r.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{r.stdout}\n{r.stderr}")


def _p(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


_LAYER_ARGS = [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _F]


class _Lib:
    prefix = ""

    def __init__(self, path: Path):
        if not path.exists():
            raise FileNotFoundError(f"{path} is not built (make -C oracle)")
        self.lib = C.CDLL(str(path))
        f = self._fn
        f("attn_block", None, [_P, _SZ, _P, _P, _I, _SZ, _SZ, _SZ, _SZ, _F, _P, _P])
        f("attn_merge", None, [_P, _P, _SZ, _SZ])
        f("attn_finish", None, [_P, _SZ, _P, _SZ, _SZ])
        f("attn_span", None, [_I, _I, _I, _I, C.POINTER(_I), C.POINTER(_I)])
        f("bf16_round", None, [_P, _P, _SZ])
        f("rope", None, [_P, _I, _I, _I, _F, _F, _I])
        f("rope_ff", None, [_P, _I, _I, _I, _F, _F, _I, _P])
        f("rmsnorm_groups", None, [_P, _SZ, _SZ, _F])
        f("rmsnorm_gamma", None, [_P, _SZ, _SZ, _P, _F])
        f("rmsnorm_plain", None, [_P, _SZ, _SZ, _F])
        f("mul_sigmoid", None, [_P, _P, _SZ])
        f("quantize_q8_0", None, [_P, _P, _P, _SZ])
        f("quantize_q4_s", None, [_P, _P, _P, _P, _SZ])
        f("block_sums", None, [_P, _P, _SZ])
        _U32 = C.c_uint32
        f("gemv_bf16", None, [_P, _P, _SZ, _P, _SZ, _U32, _U32, _U32])
        f("gemv_bf16_argmax", _I, [_P, _P, _U32, _U32])
        if self.prefix == "orc_":
            f("argmax_f32", _I, [_P, _U32])
        f("gemv_q8_0", None, [_P, _P, _P, _SZ, _P, _SZ, _U32, _U32, _U32])
        f("gemv_q4_s", None, [_P, _P, _P, _P, _SZ, _P, _SZ, _P, _SZ, _U32, _U32, _U32])

    def _fn(self, name, res, args):
        fn = getattr(self.lib, self.prefix + name)
        fn.restype = res
        fn.argtypes = args
        setattr(self, "_" + name, fn)
        return fn

    # -- the op's pieces --------------------------------------------------------------
    def attn_block(self, q, K, V, kv_bf16, kv_stride, n_keys, head_dim, n_heads, scale, q_stride=None):
        """One block's partial [n_heads, head_dim + 2] (o, m, l)."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        scores = np.zeros(n_heads * max(n_keys, 1), dtype=np.float32)
        part = np.zeros(n_heads * (head_dim + 2), dtype=np.float32)
        self._attn_block(_p(q), q_stride or head_dim, _p(K), _p(V), int(kv_bf16), kv_stride, n_keys, head_dim,
                         n_heads, scale, _p(scores), _p(part))
        return part.reshape(n_heads, head_dim + 2)

    def attn_merge(self, acc, part, head_dim, n_heads):
        acc = np.ascontiguousarray(acc, dtype=np.float32).copy()
        part = np.ascontiguousarray(part, dtype=np.float32)
        self._attn_merge(_p(acc), _p(part), head_dim, n_heads)
        return acc

    def attn_finish(self, acc, head_dim, n_heads):
        acc = np.ascontiguousarray(acc, dtype=np.float32)
        out = np.zeros(n_heads * head_dim, dtype=np.float32)
        self._attn_finish(_p(out), head_dim, _p(acc), head_dim, n_heads)
        return out.reshape(n_heads, head_dim)

    def attn_span(self, causal, window, pos, n_seq):
        a, b = _I(), _I()
        self._attn_span(int(causal), window, pos, n_seq, C.byref(a), C.byref(b))
        return a.value, b.value

    def bf16_round(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(x.shape, dtype=np.uint16)
        self._bf16_round(_p(x), _p(y), x.size)
        return y

    def rope(self, x, n_heads, head_dim, n_rot, pos, base, mode):
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        self._rope(_p(x), n_heads, head_dim, n_rot, pos, base, mode)
        return x

    def rmsnorm_groups(self, x, dim, eps=1e-6):
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        self._rmsnorm_groups(_p(x), x.size // dim, dim, eps)
        return x

    def rope_ff(self, x, n_heads, head_dim, n_rot, pos, base, mode, freq_factors=None):
        """RoPE with per-pair frequency factors (None: none)."""
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        self._rope_ff(_p(x), n_heads, head_dim, n_rot, pos, base, mode, _p(ff))
        return x

    def rmsnorm_gamma(self, x, dim, gamma=None, eps=1e-6):
        """Per-group RMSNorm with a learned gamma (None: ones)."""
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        g = np.ones(dim, np.float32) if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
        self._rmsnorm_gamma(_p(x), x.size // dim, dim, _p(g), eps)
        return x

    def rmsnorm_plain(self, x, dim, eps=1e-6):
        """Per-group RMSNorm without gamma (the V norm of Gemma 4)."""
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        self._rmsnorm_plain(_p(x), x.size // dim, dim, eps)
        return x

    # -- the weight gemvs on either side of attention ----------------------------------
    def quantize_q8_0(self, w):
        """fp32 weights [rows, cols] -> (qs int8 [rows, cols], scales bf16 bits [rows, cols/32])."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        qs = np.empty(w.shape, np.int8)
        sc = np.empty(w.shape[:-1] + (w.shape[-1] // 32,), np.uint16)
        self._quantize_q8_0(_p(w), _p(qs), _p(sc), w.size)
        return qs, sc

    def quantize_q4_s(self, w):
        """fp32 weights [rows, cols] -> (qs uint8 [rows, cols/2], scales, biases bf16 bits [rows, cols/32])."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        qs = np.empty(w.shape[:-1] + (w.shape[-1] // 2,), np.uint8)
        sc = np.empty(w.shape[:-1] + (w.shape[-1] // 32,), np.uint16)
        bi = np.empty_like(sc)
        self._quantize_q4_s(_p(w), _p(qs), _p(sc), _p(bi), w.size)
        return qs, sc, bi

    def block_sums(self, x):
        """Per-32 block sums of each row of x [n, cols]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty(x.shape[:-1] + (x.shape[-1] // 32,), np.float32)
        for i in range(x.size // x.shape[-1]):
            self._block_sums(_p(x.reshape(-1, x.shape[-1])[i]), _p(out.reshape(-1, out.shape[-1])[i]), x.shape[-1])
        return out

    def gemv_bf16(self, W, X):
        """Y [n, rows] = X [n, cols] . W^T for BF16 bits W [rows, cols]."""
        W = np.ascontiguousarray(W, dtype=np.uint16)
        X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, W.shape[1])
        Y = np.zeros((X.shape[0], W.shape[0]), np.float32)
        self._gemv_bf16(_p(W), _p(X), W.shape[1], _p(Y), W.shape[0], W.shape[0], W.shape[1], X.shape[0])
        return Y

    def gemv_bf16_argmax(self, W, x):
        """argmax_r (W . x)[r] for BF16 bits W [rows, cols] (greedy decode's
        lm_head): -1 when W is empty."""
        W = np.ascontiguousarray(W, dtype=np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        return int(self._gemv_bf16_argmax(_p(W), _p(x), W.shape[0], W.shape[1] if W.ndim == 2 else 0))

    def argmax_f32(self, y):
        """The quantised lm_head's scan over logits y (oracle only)."""
        y = np.ascontiguousarray(y, dtype=np.float32).reshape(-1)
        return int(self._argmax_f32(_p(y), y.size))

    def gemv_q8_0(self, qs, scales, X):
        qs = np.ascontiguousarray(qs, dtype=np.int8)
        scales = np.ascontiguousarray(scales, dtype=np.uint16)
        X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, qs.shape[1])
        Y = np.zeros((X.shape[0], qs.shape[0]), np.float32)
        self._gemv_q8_0(_p(qs), _p(scales), _p(X), qs.shape[1], _p(Y), qs.shape[0], qs.shape[0], qs.shape[1],
                        X.shape[0])
        return Y

    def gemv_q4_s(self, qs, scales, biases, X, xsum=None):
        qs = np.ascontiguousarray(qs, dtype=np.uint8)
        cols = qs.shape[1] * 2
        X = np.ascontiguousarray(X, dtype=np.float32).reshape(-1, cols)
        xsum = self.block_sums(X) if xsum is None else np.ascontiguousarray(xsum, dtype=np.float32)
        Y = np.zeros((X.shape[0], qs.shape[0]), np.float32)
        self._gemv_q4_s(_p(qs), _p(np.ascontiguousarray(scales, dtype=np.uint16)),
                        _p(np.ascontiguousarray(biases, dtype=np.uint16)), _p(X), cols, _p(xsum), cols // 32, _p(Y),
                        qs.shape[0], qs.shape[0], cols, X.shape[0])
        return Y

    def mul_sigmoid(self, y, g):
        """y * sigmoid(g), elementwise (Qwen3.5's output gate)."""
        y = np.ascontiguousarray(y, dtype=np.float32).copy()
        g = np.ascontiguousarray(g, dtype=np.float32)
        assert g.size == y.size
        self._mul_sigmoid(_p(y), _p(g), y.size)
        return y


def _layer_call(fn, extra, q, K, V, kv_bf16, rows, pos0, n_seq, window, causal, n_head, n_kv, head_dim, scale):
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_tok = q.size // (n_head * head_dim)
    out = np.zeros((n_tok, n_head * head_dim), dtype=np.float32)
    if n_seq is None:
        n_seq = pos0 + n_tok
    K = np.ascontiguousarray(K)
    V = np.ascontiguousarray(V)
    rc = fn(_p(q), _p(out), _p(K), _p(V), int(kv_bf16), rows, n_tok, pos0, n_seq, window, int(causal), n_head, n_kv,
            head_dim, scale, *extra)
    if rc not in (None, 0):
        raise ValueError("oracle refused the arguments")
    return out


class Oracle(_Lib):
    """This repository's C++ restatement of nnc's attention core."""

    prefix = "orc_"

    def __init__(self, path: Path = ORACLE_SO):
        super().__init__(path)
        self._fn("attend_layer", _I, _LAYER_ARGS + [_I])
        self._fn("textbook_attend", None, _LAYER_ARGS)
        self._fn("kv_rows", _I, [_I, _I, _I])
        self._fn("max_rewind", _I, [_I, _I])
        self._fn("f32_from_bf16", _F, [C.c_uint16])
        self._fn("bf16_from_f32", C.c_uint16, [_F])
        self._fn("ref_fixture_attn_blocks", _I, [_I, _P, _P, _P])
        self._fn("prep_append", None, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _F, _I, _F, _F, _I, _P, _I, _I, _I, _P,
                                       _P])

    def attend_layer(self, q, K, V, *, kv_bf16, rows, pos0, n_seq=None, window=0, causal=True, n_head, n_kv,
                     head_dim, scale, threads=8):
        """Layer-granularity attention: nnc's dispatch over this file's kernels."""
        return _layer_call(self._attend_layer, [threads], q, K, V, kv_bf16, rows, pos0, n_seq, window, causal,
                           n_head, n_kv, head_dim, scale)

    def textbook(self, q, K, V, *, kv_bf16, rows, pos0, n_seq=None, window=0, causal=True, n_head, n_kv, head_dim,
                 scale):
        """Double-precision softmax attention per query head over its span."""
        return _layer_call(self._textbook_attend, [], q, K, V, kv_bf16, rows, pos0, n_seq, window, causal, n_head,
                           n_kv, head_dim, scale)

    def prep_append(self, q, k, v, K, V, *, n_head, n_kv, head_dim, pos0, kv_bf16, q_gamma=None, k_gamma=None,
                    v_norm=False, eps=1e-6, n_rot=0, base=10000.0, pos_scale=1.0, mode=0, freq_factors=None):
        """Per-head norms, RoPE and the K/V append of one batch (reference
        model.cpp:1616-1691). q, k, v: [n_tok][heads * head_dim] fp32; K, V: the
        layer's buffers ([rows][kv_dim], uint16 BF16 bits or fp32), copied and
        returned with the new rows. Returns (q, K, V)."""
        q = np.ascontiguousarray(q, dtype=np.float32).copy()
        k = np.ascontiguousarray(k, dtype=np.float32).copy()
        v = np.ascontiguousarray(v, dtype=np.float32).copy()
        K = np.ascontiguousarray(K).copy()
        V = np.ascontiguousarray(V).copy()
        n_tok = q.size // (n_head * head_dim)
        qg = None if q_gamma is None else np.ascontiguousarray(q_gamma, dtype=np.float32)
        kg = None if k_gamma is None else np.ascontiguousarray(k_gamma, dtype=np.float32)
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        self._prep_append(_p(q), _p(k), _p(v), n_tok, n_head, n_kv, head_dim, _p(qg), _p(kg), int(v_norm), eps, n_rot,
                          base, pos_scale, mode, _p(ff), pos0, K.shape[0], int(kv_bf16), _p(K), _p(V))
        return q, K, V

    def kv_rows(self, n_ctx, window, n_batch):
        return self._kv_rows(n_ctx, window, n_batch)

    def max_rewind(self, rows, window):
        return self._max_rewind(rows, window)

    def ref_fixture_attn_blocks(self, which):
        """Inputs of case `which` of the reference's test_nnc_attn_blocks."""
        q = np.zeros(3 * 64, dtype=np.float32)
        K = np.zeros(600 * 2 * 64, dtype=np.float32)
        V = np.zeros(600 * 2 * 64, dtype=np.float32)
        hd = self._ref_fixture_attn_blocks(which, _p(q), _p(K), _p(V))
        if hd < 0:
            raise ValueError(which)
        return hd, q[: 3 * hd], K[: 600 * 2 * hd].reshape(600, 2 * hd), V[: 600 * 2 * hd].reshape(600, 2 * hd)


class Reference(_Lib):
    """The reference's own compiled attention kernels, thread pool and helpers."""

    prefix = "ref_"

    def __init__(self, path: Path = REF_SO):
        super().__init__(path)
        self._fn("attend_layer", _I, _LAYER_ARGS)
        self._fn("set_threads", None, [_I])
        self._fn("threads", _I, [])

    def set_threads(self, n: int) -> None:
        self._set_threads(n)

    def threads(self) -> int:
        return self._threads()

    def attend_layer(self, q, K, V, *, kv_bf16, rows, pos0, n_seq=None, window=0, causal=True, n_head, n_kv,
                     head_dim, scale):
        """nnc_attn_block/merge/finish through nnc's own worker pool, with the
        dispatch of reference model.cpp:1229-1317, 1693-1757 restated."""
        return _layer_call(self._attend_layer, [], q, K, V, kv_bf16, rows, pos0, n_seq, window, causal, n_head, n_kv,
                           head_dim, scale)


def reference_available() -> bool:
    return REF_SO.exists()

"""Python host side of libnnc_hip.so (include/nnc_hip.h) through ctypes.

The library is the product; this module only binds it. It mirrors the pieces
of nnc's interface around the attention op:

- ``NncStatus`` / ``NncError``: nnc's status codes and its "status plus
  thread-local message" error convention (reference src/libnnc/nnc.h:50-61,
  nnc.cpp:24-43);
- ``kv_rows`` / ``max_rewind``: the K/V buffer sizing rule of model_kv_init
  (reference src/libnnc/model.cpp:1936-1957);
- ``attn_span``: model_attn_span (reference src/libnnc/model.cpp:2300-2316);
- ``bf16_round`` / ``bf16_to_f32``: nnc_f32_to_bf16 / nnc_bf16_to_f32
  (reference src/libnnc/runtime.h:97-113), vectorised;
- ``KVCache``: one session's device K/V buffers (model_kv_cache::bufs,
  reference src/libnnc/model.h:252-326) with the append of reference
  model.cpp:1662-1691 and the per-layer attention call that replaces the
  attention core of reference model.cpp:1693-1761.

Loading fails loudly when the library has not been built: there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes as C
import enum
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libnnc_hip.so"
ATTN_BLOCK = 256  # keys per block (reference model.h:229)


class NncStatus(enum.IntEnum):
    OK = 0
    INVALID_ARGUMENT = 1
    UNSUPPORTED_CPU = 2
    IO = 3
    BAD_FORMAT = 4
    UNSUPPORTED_MODEL = 5
    OUT_OF_MEMORY = 6
    CONTEXT_FULL = 7
    CANCELLED = 8


class NncError(RuntimeError):
    """A call returned a status other than NNC_OK; `message` is the library's
    nnc_hip_last_error() text for it."""

    def __init__(self, status: int, message: str):
        self.status = NncStatus(status)
        self.message = message
        super().__init__(f"{self.status.name.lower()}: {message}")


_lib = None

_P = C.c_void_p
_I = C.c_int32
_F = C.c_float
_B = C.c_bool
_U64 = C.c_uint64

class NncHipGemvMat(C.Structure):
    """nnc_hip_gemv_mat: one matrix of a gemv group."""
    _fields_ = [("w", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("y", C.c_void_p),
                ("y_stride", C.c_size_t), ("rows", C.c_uint32)]


GEMV_FORMATS = {"bf16": 0, "q8_0": 1, "q4_s": 2}


class NncHipPrep(C.Structure):
    """struct nnc_hip_prep of include/nnc_hip.h (pointers are device addresses)."""

    _fields_ = [("n_head", _I), ("n_kv", _I), ("head_dim", _I), ("q_gamma", _P), ("k_gamma", _P), ("v_norm", _I),
                ("rms_eps", _F), ("n_rot", _I), ("freq_base", _F), ("pos_scale", _F), ("rope_mode", _I),
                ("freq_factors", _P)]


# nnc_hip_log_callback: (level, message, user)
LOG_CALLBACK = C.CFUNCTYPE(None, C.c_int, C.c_char_p, C.c_void_p)

# name: (restype, argtypes) for every function include/nnc_hip.h declares.
SIGNATURES = {
    "nnc_hip_set_log_callback": (None, [LOG_CALLBACK, _P]),
    "nnc_hip_kv_create": (C.c_int, [_I, C.POINTER(_I), C.POINTER(_I), _B, C.POINTER(_P)]),
    "nnc_hip_kv_free": (None, [_P]),
    "nnc_hip_kv_bytes": (_U64, [_P]),
    "nnc_hip_kv_set_exact_batches": (C.c_int, [_P, _B]),
    "nnc_hip_kv_append": (C.c_int, [_P, _I, _I, _I, _P, _P]),
    "nnc_hip_kv_append_f32": (C.c_int, [_P, _I, _I, _I, _P, _P]),
    "nnc_hip_kv_append_f32_device": (C.c_int, [_P, _I, _I, _I, _P, _P]),
    "nnc_hip_kv_prep_append_device": (C.c_int, [_P, _I, _I, _I, _P, _P, _P, C.POINTER(NncHipPrep)]),
    "nnc_hip_kv_read": (C.c_int, [_P, _I, _I, _I, _P, _P]),
    "nnc_hip_attend": (C.c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _B, _I, _I, _I, _F]),
    "nnc_hip_attend_device": (C.c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _B, _I, _I, _I, _F]),
    "nnc_hip_attend_device_noalloc": (C.c_int, [_P, _I, _P, _P, _I, _I, _I, _I, _B, _I, _I, _I, _F]),
    "nnc_hip_attend_gated": (C.c_int, [_P, _I, _P, _P, _P, _I, _I, _I, _I, _B, _I, _I, _I, _F]),
    "nnc_hip_attend_gated_device": (C.c_int, [_P, _I, _P, _P, _P, _I, _I, _I, _I, _B, _I, _I, _I, _F]),
    "nnc_hip_gemv_bf16": (C.c_int, [_P, _P, _P, C.c_size_t, _P, C.c_size_t, C.c_uint32, C.c_uint32, C.c_uint32]),
    "nnc_hip_gemv_bf16_argmax": (C.c_int, [_P, _P, _P, C.c_uint32, C.c_uint32, C.POINTER(C.c_int32)]),
    "nnc_hip_argmax_f32": (C.c_int, [_P, _P, C.c_uint32, C.POINTER(C.c_int32)]),
    "nnc_hip_gemv_q8_0": (C.c_int, [_P, _P, _P, _P, C.c_size_t, _P, C.c_size_t, C.c_uint32, C.c_uint32, C.c_uint32]),
    "nnc_hip_gemv_group": (C.c_int, [_P, C.c_int32, C.c_int32, C.POINTER(NncHipGemvMat), _P, C.c_size_t, _P,
                                     C.c_size_t, C.c_uint32, C.c_uint32]),
    "nnc_hip_gemv_q4_s": (C.c_int, [_P, _P, _P, _P, _P, C.c_size_t, _P, C.c_size_t, _P, C.c_size_t, C.c_uint32,
                                    C.c_uint32, C.c_uint32]),
    "nnc_hip_kv_sync": (C.c_int, [_P]),
    "nnc_hip_kv_stream": (_P, [_P]),
    "nnc_hip_fill_normal": (C.c_int, [_P, _U64, _U64, _I, _B, _P]),
    "nnc_hip_last_error": (C.c_char_p, []),
    "nnc_hip_status_string": (C.c_char_p, [C.c_int]),
}


def load_library(path: Path | str | None = None) -> C.CDLL:
    """Loads libnnc_hip.so (built by libllmcpu_amd.build) and binds its C ABI.
    Raises FileNotFoundError when it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the attention op has no CPU fallback)"
        )
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


_log_keep = None  # the installed callback object (ctypes needs it alive)


def set_log_callback(fn) -> None:
    """Routes the bridge's log lines to fn(level, message) (levels as nnc's:
    0 debug, 1 info, 2 warn, 3 error); None restores the default (warnings
    and errors to stderr)."""
    global _log_keep
    lib = load_library()
    if fn is None:
        _log_keep = None
        lib.nnc_hip_set_log_callback(LOG_CALLBACK(), None)
        return
    _log_keep = LOG_CALLBACK(lambda level, msg, user: fn(int(level), msg.decode("utf-8", "replace")))
    lib.nnc_hip_set_log_callback(_log_keep, None)


def _check(status: int) -> None:
    if status != NncStatus.OK:
        raise NncError(status, load_library().nnc_hip_last_error().decode("utf-8", "replace"))


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None else a.ctypes.data


# ---- host rules mirrored from nnc --------------------------------------------------

def kv_rows(n_ctx: int, window: int, n_batch: int) -> int:
    """Rows of a layer's K/V buffer: a ring of round_up(window + n_batch, 256)
    rows for a sliding layer when that is smaller than the context, else n_ctx
    (reference model.cpp:1936-1957)."""
    nb = n_batch if n_batch > 0 else 1
    ring = (window + nb + ATTN_BLOCK - 1) // ATTN_BLOCK * ATTN_BLOCK
    return ring if (window > 0 and ring < n_ctx) else n_ctx


def max_rewind(rows: int, window: int) -> int:
    """How far below the highest written position a ring may go back
    (reference model.cpp:1949)."""
    return rows - window


def attn_span(causal: bool, window: int, pos: int, n_seq: int) -> tuple[int, int]:
    """(first, last) key position that position `pos` attends to
    (reference model.cpp:2300-2316)."""
    if causal:
        first = pos + 1 - window if (window > 0 and pos + 1 > window) else 0
        return first, min(pos, n_seq - 1)
    if window > 0:
        return max(0, pos - window // 2), min(n_seq - 1, pos + window // 2)
    return 0, n_seq - 1


def bf16_round(x: np.ndarray) -> np.ndarray:
    """F32 -> BF16 bits with round-to-nearest-even on the bit pattern, the
    formula of nnc_f32_to_bf16 (reference runtime.h:106-113)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    """BF16 bits -> F32 by a 16-bit shift (reference runtime.h:97-103)."""
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- the device cache ----------------------------------------------------------------

class KVCache:
    """A session's K/V buffers in HBM. `rows[i]` and `kv_dim[i]` size buffer i
    as model_kv_init would; `bf16` picks the element type (nnc_kv_type)."""

    def __init__(self, rows: list[int], kv_dim: list[int], bf16: bool = True):
        lib = load_library()
        n = len(rows)
        if len(kv_dim) != n:
            raise ValueError("rows and kv_dim differ in length")
        r = (_I * n)(*rows)
        d = (_I * n)(*kv_dim)
        h = _P()
        _check(lib.nnc_hip_kv_create(n, r, d, bool(bf16), C.byref(h)))
        self._lib = lib
        self.handle = h
        self.rows = list(rows)
        self.kv_dim = list(kv_dim)
        self.bf16 = bool(bf16)

    def close(self) -> None:
        if self.handle:
            self._lib.nnc_hip_kv_free(self.handle)
            self.handle = _P()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def nbytes(self) -> int:
        return int(self._lib.nnc_hip_kv_bytes(self.handle))

    @property
    def stream(self) -> int:
        return int(self._lib.nnc_hip_kv_stream(self.handle) or 0)

    def set_exact_batches(self, exact: bool) -> None:
        """Batches over 16 tokens on the split-K path too, each token with the
        bits of its one-token call (default False: the prefill kernel)."""
        _check(self._lib.nnc_hip_kv_set_exact_batches(self.handle, bool(exact)))

    def append(self, buf: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        """Rows already in the cache's element type: uint16 BF16 bits, or float32."""
        dt = np.uint16 if self.bf16 else np.float32
        k = np.ascontiguousarray(k, dtype=dt)
        v = np.ascontiguousarray(v, dtype=dt)
        n_tok = k.size // self.kv_dim[buf] if 0 <= buf < len(self.kv_dim) else 0
        _check(self._lib.nnc_hip_kv_append(self.handle, buf, pos0, n_tok, _ptr(k), _ptr(v)))
        self.sync()

    def append_f32(self, buf: int, pos0: int, k: np.ndarray, v: np.ndarray) -> None:
        """F32 rows; a BF16 cache rounds them on the device (nnc_f32_to_bf16 bits)."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        n_tok = k.size // self.kv_dim[buf] if 0 <= buf < len(self.kv_dim) else 0
        _check(self._lib.nnc_hip_kv_append_f32(self.handle, buf, pos0, n_tok, _ptr(k), _ptr(v)))
        self.sync()

    def read(self, buf: int, row0: int, n_rows: int) -> tuple[np.ndarray, np.ndarray]:
        dt = np.uint16 if self.bf16 else np.float32
        d = self.kv_dim[buf]
        k = np.empty((n_rows, d), dtype=dt)
        v = np.empty((n_rows, d), dtype=dt)
        _check(self._lib.nnc_hip_kv_read(self.handle, buf, row0, n_rows, _ptr(k), _ptr(v)))
        return k, v

    def attend(self, buf: int, q: np.ndarray, *, pos0: int, n_seq: int | None = None, window: int = 0,
               causal: bool = True, n_head: int, n_kv: int, head_dim: int, scale: float,
               gate: np.ndarray | None = None) -> np.ndarray:
        """Attention of q [n_tok, n_head*head_dim] (float32) over buffer `buf`;
        returns out of the same shape. With `gate` (same shape), out is scaled
        by sigmoid(gate) as Qwen3.5 does."""
        q = np.ascontiguousarray(q, dtype=np.float32)
        n_tok = q.size // (n_head * head_dim)
        out = np.empty((n_tok, n_head * head_dim), dtype=np.float32)
        if n_seq is None:
            n_seq = pos0 + n_tok
        if gate is None:
            _check(self._lib.nnc_hip_attend(self.handle, buf, _ptr(q), _ptr(out), n_tok, pos0, n_seq, window,
                                            bool(causal), n_head, n_kv, head_dim, float(scale)))
        else:
            gate = np.ascontiguousarray(gate, dtype=np.float32)
            if gate.size != q.size:
                raise ValueError(f"gate has {gate.size} values, q {q.size}")
            _check(self._lib.nnc_hip_attend_gated(self.handle, buf, _ptr(q), _ptr(gate), _ptr(out), n_tok, pos0,
                                                  n_seq, window, bool(causal), n_head, n_kv, head_dim,
                                                  float(scale)))
        return out

    def attend_device(self, buf: int, q_dev: int, out_dev: int, *, n_tok: int, pos0: int, n_seq: int | None = None,
                      window: int = 0, causal: bool = True, n_head: int, n_kv: int, head_dim: int,
                      scale: float) -> None:
        """As attend with device addresses; queued on the cache's stream."""
        if n_seq is None:
            n_seq = pos0 + n_tok
        _check(self._lib.nnc_hip_attend_device(self.handle, buf, q_dev, out_dev, n_tok, pos0, n_seq, window,
                                               bool(causal), n_head, n_kv, head_dim, float(scale)))

    def attend_device_noalloc(self, buf: int, q_dev: int, out_dev: int, *, n_tok: int, pos0: int,
                              n_seq: int | None = None, window: int = 0, causal: bool = True, n_head: int,
                              n_kv: int, head_dim: int, scale: float) -> None:
        """attend_device through nnc_hip_attend_device_noalloc: no device
        allocation, the decode partials in the library's fixed per-device array."""
        if n_seq is None:
            n_seq = pos0 + n_tok
        _check(self._lib.nnc_hip_attend_device_noalloc(self.handle, buf, q_dev, out_dev, n_tok, pos0, n_seq, window,
                                                       bool(causal), n_head, n_kv, head_dim, float(scale)))

    def prep_append_device(self, buf: int, q_dev: int, k_dev: int, v_dev: int, *, pos0: int, n_tok: int,
                           prep: NncHipPrep) -> None:
        """Per-head norms, RoPE and the K/V append of a batch whose q/k/v are in
        device memory (q updated in place); queued on the cache's stream."""
        _check(self._lib.nnc_hip_kv_prep_append_device(self.handle, buf, pos0, n_tok, q_dev, k_dev, v_dev,
                                                       C.byref(prep)))

    def prep_append(self, buf: int, q: np.ndarray, k: np.ndarray, v: np.ndarray, *, pos0: int, n_head: int, n_kv: int,
                    head_dim: int, q_gamma: np.ndarray | None = None, k_gamma: np.ndarray | None = None,
                    v_norm: bool = False, eps: float = 1e-6, n_rot: int = 0, base: float = 10000.0,
                    pos_scale: float = 1.0, mode: int = 0, freq_factors: np.ndarray | None = None) -> np.ndarray:
        """prep_append_device from host arrays (q, k, v and the gammas uploaded
        to scratch device memory, freed afterwards; the frequency factors stay
        in host memory); returns the normalised, rotated q."""
        from . import hip_rt

        q = np.ascontiguousarray(q, dtype=np.float32)
        arrays = [q, np.ascontiguousarray(k, dtype=np.float32), np.ascontiguousarray(v, dtype=np.float32)]
        extras = [q_gamma, k_gamma]
        ff = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)
        ptrs, dev = [], []
        try:
            for a in arrays + [None if e is None else np.ascontiguousarray(e, dtype=np.float32) for e in extras]:
                if a is None:
                    ptrs.append(None)
                    continue
                d = hip_rt.malloc(max(a.nbytes, 4))
                dev.append(d)
                hip_rt.to_device(d, a)
                ptrs.append(d)
            prep = NncHipPrep(n_head, n_kv, head_dim, ptrs[3], ptrs[4], int(bool(v_norm)), eps, n_rot, base, pos_scale,
                              mode, None if ff is None else ff.ctypes.data)
            n_tok = q.size // (n_head * head_dim)
            self.prep_append_device(buf, ptrs[0], ptrs[1], ptrs[2], pos0=pos0, n_tok=n_tok, prep=prep)
            self.sync()
            return hip_rt.to_host(np.empty_like(q), ptrs[0])
        finally:
            for d in dev:
                hip_rt.free(d)

    # -- the weight gemvs, with this cache as the execution context ------------------
    def gemv_device(self, fmt: str, w: tuple, x_dev: int, y_dev: int, *, rows: int, cols: int, n_batch: int,
                    x_stride: int | None = None, y_stride: int | None = None, xsum_dev: int = 0,
                    xsum_stride: int = 0) -> None:
        """Y = W . X on device memory: fmt "bf16" (w = (W,)), "q8_0" (w = (qs, scales))
        or "q4_s" (w = (qs, scales, biases)), each a device address; queued on the
        cache's stream."""
        xs = cols if x_stride is None else x_stride
        ys = rows if y_stride is None else y_stride
        if fmt == "bf16":
            st = self._lib.nnc_hip_gemv_bf16(self.handle, w[0], x_dev, xs, y_dev, ys, rows, cols, n_batch)
        elif fmt == "q8_0":
            st = self._lib.nnc_hip_gemv_q8_0(self.handle, w[0], w[1], x_dev, xs, y_dev, ys, rows, cols, n_batch)
        elif fmt == "q4_s":
            st = self._lib.nnc_hip_gemv_q4_s(self.handle, w[0], w[1], w[2], x_dev, xs, xsum_dev or None,
                                             xsum_stride, y_dev, ys, rows, cols, n_batch)
        else:
            raise ValueError(f"unknown weight format {fmt!r}")
        _check(st)

    def gemv_group_device(self, fmt: str, mats: list, x_dev: int, *, cols: int, n_batch: int,
                          x_stride: int | None = None, xsum_dev: int = 0, xsum_stride: int = 0) -> None:
        """Several gemvs over the same X in one launch: mats is a list of (w, y_dev,
        rows) or (w, y_dev, rows, y_stride) with w as in gemv_device; queued on
        the cache's stream."""
        arr = (NncHipGemvMat * max(1, len(mats)))()
        for i, m in enumerate(mats):
            w, y_dev, rows = m[0], m[1], m[2]
            ys = m[3] if len(m) > 3 else rows
            w = tuple(w) + (None,) * (3 - len(w))
            arr[i] = NncHipGemvMat(w[0], w[1], w[2], y_dev, ys, rows)
        if fmt not in GEMV_FORMATS:
            raise ValueError(f"unknown weight format {fmt!r}")
        _check(self._lib.nnc_hip_gemv_group(self.handle, GEMV_FORMATS[fmt], len(mats), arr, x_dev,
                                            cols if x_stride is None else x_stride, xsum_dev or None, xsum_stride,
                                            cols, n_batch))

    def gemv(self, fmt: str, w: tuple, x: np.ndarray, *, rows: int, cols: int,
             xsum: np.ndarray | None = None) -> np.ndarray:
        """gemv_device from host arrays (uploaded to scratch device memory,
        freed afterwards); returns Y [n_batch, rows]."""
        from . import hip_rt

        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, cols)
        n = x.shape[0]
        arrays = [np.ascontiguousarray(a) for a in w] + [x] + ([] if xsum is None else
                                                               [np.ascontiguousarray(xsum, dtype=np.float32)])
        dev = []
        try:
            for a in arrays:
                d = hip_rt.malloc(max(a.nbytes, 16))
                dev.append(d)
                hip_rt.to_device(d, a)
            y_dev = hip_rt.malloc(n * rows * 4)
            dev.append(y_dev)
            nw = len(w)
            self.gemv_device(fmt, tuple(dev[:nw]), dev[nw], y_dev, rows=rows, cols=cols, n_batch=n,
                             xsum_dev=dev[nw + 1] if xsum is not None else 0, xsum_stride=cols // 32)
            self.sync()
            return hip_rt.to_host(np.empty((n, rows), np.float32), y_dev)
        finally:
            for d in dev:
                hip_rt.free(d)

    def gemv_argmax_device(self, w_dev: int, x_dev: int, *, rows: int, cols: int) -> int:
        """argmax_r (W . x)[r] for BF16 W on the device (the lm_head of greedy
        decode; nnc_gemv_bf16w_argmax_f32x); waits for the cache's stream."""
        idx = C.c_int32(-2)
        _check(self._lib.nnc_hip_gemv_bf16_argmax(self.handle, w_dev, x_dev, rows, cols, C.byref(idx)))
        return int(idx.value)

    def gemv_argmax(self, w: np.ndarray, x: np.ndarray) -> int:
        """gemv_argmax_device from host arrays (BF16 bits w [rows, cols], x [cols])."""
        from . import hip_rt

        w = np.ascontiguousarray(w, dtype=np.uint16)
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        dev = []
        try:
            for a in (w, x):
                d = hip_rt.malloc(max(a.nbytes, 16))
                dev.append(d)
                hip_rt.to_device(d, a)
            return self.gemv_argmax_device(dev[0], dev[1], rows=w.shape[0], cols=w.shape[1])
        finally:
            for d in dev:
                hip_rt.free(d)

    def argmax(self, y: np.ndarray) -> int:
        """nnc_hip_argmax_f32 of host logits y (uploaded to scratch device memory)."""
        from . import hip_rt

        y = np.ascontiguousarray(y, dtype=np.float32).reshape(-1)
        d = hip_rt.malloc(max(y.nbytes, 16))
        try:
            hip_rt.to_device(d, y)
            idx = C.c_int32(-2)
            _check(self._lib.nnc_hip_argmax_f32(self.handle, d, y.size, C.byref(idx)))
            return int(idx.value)
        finally:
            hip_rt.free(d)

    def sync(self) -> None:
        _check(self._lib.nnc_hip_kv_sync(self.handle))


def fill_normal(dst: int, n: int, seed: int, norm_dim: int = 0, bf16: bool = False, stream: int = 0) -> None:
    """Device-side N(0,1) fill (splitmix64 + Box-Muller), optionally
    RMS-normalised per run of norm_dim, stored as F32 or BF16."""
    _check(load_library().nnc_hip_fill_normal(dst, n, seed, norm_dim, bool(bf16), stream or None))

"""Synthetic inputs at the benchmark's model shapes.

Generator: splitmix64 (Steele, Lea and Flood, 2014) as a counter-based stream,
element i of stream `seed` drawn by Box-Muller from draws 2*(i//2) and
2*(i//2)+1 (cosine branch for even i, sine for odd i). The device fill of
libnnc_hip.so (nnc_hip_fill_normal) uses the same formula, so host and device
inputs agree to the last few bits of libm. It is portable, unlike
std::normal_distribution, whose algorithm differs between C++ libraries.

Seeds: stream (base_seed + 1000 * config + layer) * 256 + tensor, tensor 0/1/2
for Q/K/V, layers independent.

Q/K preparation mirrors what nnc does to them before attention:
- RoPE (reference src/libnnc/nn_ops.cpp:1830-1873): angle_i = pos *
  base^(-2i/n_rot), the per-step ratio accumulated in fp32; NORM mode pairs
  lanes 2i and 2i+1 (Llama, reference model.cpp:641), NEOX pairs i and
  i + n_rot/2;
- per-head RMSNorm with gamma = 1 (Qwen3's Q/K norms, reference
  model.cpp:1619-1641 and nn_ops.cpp:590-632).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from .nnc_hip import bf16_round, kv_rows

BASE_SEED = 1234
_GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def stream_seed(config: int, layer: int, tensor: int) -> int:
    return ((BASE_SEED + 1000 * config + layer) * 256 + tensor) & 0xFFFFFFFFFFFFFFFF


def _splitmix64(seed: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx + np.uint64(1)) * _GAMMA
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def normal(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Elements start .. start + n - 1 of the N(0,1) stream `seed`, float32."""
    if n <= 0:
        return np.empty(0, dtype=np.float32)
    p0, p1 = start // 2, (start + n + 1) // 2
    pair = np.arange(p0, p1, dtype=np.uint64)
    a = _splitmix64(seed, np.uint64(2) * pair)
    b = _splitmix64(seed, np.uint64(2) * pair + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    r = np.sqrt(-2.0 * np.log(u1))
    th = 2.0 * math.pi * u2
    out = np.empty(2 * (p1 - p0), dtype=np.float64)
    out[0::2] = r * np.cos(th)
    out[1::2] = r * np.sin(th)
    off = start - 2 * p0
    return out[off:off + n].astype(np.float32)


def rope(x: np.ndarray, pos: np.ndarray, head_dim: int, base: float, mode: str = "norm") -> np.ndarray:
    """Rotates x [n, n_heads * head_dim] whose row j sits at position pos[j]."""
    n_rot = head_dim
    half = n_rot // 2
    ratio = np.float32(base) ** np.float32(-2.0 / n_rot)
    inv = np.empty(half, dtype=np.float32)
    v = np.float32(1.0)
    for i in range(half):
        inv[i] = v
        v = np.float32(v * ratio)
    theta = np.asarray(pos, dtype=np.float32)[:, None] * inv[None, :]
    c = np.cos(theta).astype(np.float32)[:, None, :]
    s = np.sin(theta).astype(np.float32)[:, None, :]
    n = x.shape[0]
    xh = x.reshape(n, -1, head_dim).copy()
    if mode == "norm":
        a, b = xh[..., 0:n_rot:2].copy(), xh[..., 1:n_rot:2].copy()
        xh[..., 0:n_rot:2] = c * a - s * b
        xh[..., 1:n_rot:2] = s * a + c * b
    else:
        a, b = xh[..., :half].copy(), xh[..., half:n_rot].copy()
        xh[..., :half] = c * a - s * b
        xh[..., half:n_rot] = s * a + c * b
    return xh.reshape(n, -1)


def rmsnorm_heads(x: np.ndarray, head_dim: int, eps: float = 1e-6) -> np.ndarray:
    """Per-head RMSNorm, gamma = 1; the sum of squares in double."""
    n = x.shape[0]
    xh = x.reshape(n, -1, head_dim).astype(np.float64)
    r = 1.0 / np.sqrt((xh * xh).mean(axis=-1, keepdims=True) + eps)
    return (x.reshape(n, -1, head_dim) * r.astype(np.float32)).reshape(n, -1).astype(np.float32)


@dataclass(frozen=True)
class AttnConfig:
    """One of the benchmark's model shapes (attention only)."""
    index: int
    name: str
    n_head: int
    n_kv: int
    head_dim: int
    n_layer: int
    kv_bf16: bool = True
    window: int = 0  # sliding window of the local layers
    swa_period: int = 0  # every swa_period-th layer is global: (li + 1) % period != 0 slides
    rope_theta: float = 0.0  # > 0: RoPE NORM on Q and K at their positions
    qk_norm: bool = False  # per-head RMSNorm of Q and K
    decode_ctx: tuple = ()
    prefill: tuple = ()  # (prompt tokens, chunk)
    decode_steps: int = 1
    tol: float = 5e-3  # max-abs error bound against nnc's CPU output
    scale: float = field(default=0.0)

    @property
    def group(self) -> int:
        return self.n_head // self.n_kv

    @property
    def kv_dim(self) -> int:
        return self.n_kv * self.head_dim

    @property
    def attn_scale(self) -> float:
        return self.scale if self.scale > 0 else 1.0 / math.sqrt(self.head_dim)

    def sliding(self, layer: int) -> bool:
        """Gemma 3's pattern: every swa_period-th layer is global
        (reference model.cpp:1061-1073)."""
        return self.window > 0 and self.swa_period > 0 and (layer + 1) % self.swa_period != 0

    def layer_window(self, layer: int) -> int:
        return self.window if self.sliding(layer) else 0

    def layer_rows(self, layer: int, n_ctx: int, n_batch: int) -> int:
        return kv_rows(n_ctx, self.layer_window(layer), n_batch) if self.sliding(layer) else n_ctx


CONFIGS = {
    "A": AttnConfig(0, "gemma-3-270m decode", 4, 1, 256, 18, kv_bf16=False, decode_ctx=(1024,), tol=1e-3),
    "B": AttnConfig(1, "llama-3.2-1b decode", 32, 8, 64, 16, rope_theta=500000.0, decode_ctx=(512, 4096, 16384)),
    "C": AttnConfig(2, "gemma-3-1b local/global", 4, 1, 256, 26, window=512, swa_period=6, decode_ctx=(8192,),
                    prefill=(8192, 2048)),
    "D": AttnConfig(3, "qwen3-4b", 32, 8, 128, 36, qk_norm=True, decode_ctx=(4096, 32768), prefill=(4096, 512)),
    "E": AttnConfig(4, "gemma-3-4b long context", 8, 4, 256, 34, window=1024, swa_period=6, prefill=(16384, 1024),
                    decode_steps=256),
}


def qk_rows(cfg: AttnConfig, layer: int, tensor: int, pos: np.ndarray, n_heads: int) -> np.ndarray:
    """Q (tensor 0, n_heads = n_head) or K (tensor 1, n_heads = n_kv) rows for
    positions pos, prepared as the model would: RMSNorm, then RoPE."""
    width = n_heads * cfg.head_dim
    x = _rows(stream_seed(cfg.index, layer, tensor), width, pos)
    if cfg.qk_norm:
        x = rmsnorm_heads(x, cfg.head_dim)
    if cfg.rope_theta > 0:
        x = rope(x, pos, cfg.head_dim, cfg.rope_theta, "norm")
    return x.astype(np.float32)


def _rows(seed: int, width: int, pos) -> np.ndarray:
    """Rows of `width` stream elements, row j starting at element pos[j] * width."""
    p = np.asarray(pos, dtype=np.int64)
    if len(p) == 0:
        return np.empty((0, width), np.float32)
    if np.all(np.diff(p) == 1):
        return normal(seed, width * len(p), int(p[0]) * width).reshape(len(p), width)
    return np.stack([normal(seed, width, int(q) * width) for q in p])


def v_rows(cfg: AttnConfig, layer: int, pos: np.ndarray) -> np.ndarray:
    return _rows(stream_seed(cfg.index, layer, 2), cfg.kv_dim, pos)


def kv_rows_f32(cfg: AttnConfig, layer: int, pos: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """F32 K and V rows for positions pos, as the model computes them before the append."""
    return qk_rows(cfg, layer, 1, pos, cfg.n_kv), v_rows(cfg, layer, pos)


def to_cache_dtype(cfg: AttnConfig, x: np.ndarray) -> np.ndarray:
    """The append's conversion: BF16 round-to-nearest-even, or F32 as is."""
    return bf16_round(x) if cfg.kv_bf16 else np.ascontiguousarray(x, dtype=np.float32)


def cache_buffer(cfg: AttnConfig, layer: int, rows: int, n_seq: int) -> tuple[np.ndarray, np.ndarray]:
    """A layer's K/V buffer contents after positions 0 .. n_seq - 1 were
    appended: position p in row p % rows (only the last `rows` positions
    survive in a ring). Unwritten rows are zero."""
    dt = np.uint16 if cfg.kv_bf16 else np.float32
    K = np.zeros((rows, cfg.kv_dim), dtype=dt)
    V = np.zeros((rows, cfg.kv_dim), dtype=dt)
    p0 = max(0, n_seq - rows)
    pos = np.arange(p0, n_seq)
    k, v = kv_rows_f32(cfg, layer, pos)
    K[pos % rows] = to_cache_dtype(cfg, k)
    V[pos % rows] = to_cache_dtype(cfg, v)
    return K, V

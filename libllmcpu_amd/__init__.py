"""nnc's attention hot path (causal GQA softmax(Q K^T * scale) V over nnc's
K/V cache: decode, chunked prefill, sliding-window layers) on one AMD Instinct
MI355X. The compute lives in libnnc_hip.so (hand-written gfx950 HIP kernels
behind the C ABI of include/nnc_hip.h); this package binds it, builds it, and
generates the benchmark's synthetic inputs."""
from .nnc_hip import (  # noqa: F401
    ATTN_BLOCK,
    KVCache,
    NncError,
    NncHipPrep,
    NncStatus,
    attn_span,
    bf16_round,
    bf16_to_f32,
    fill_normal,
    kv_rows,
    load_library,
    max_rewind,
    set_log_callback,
)

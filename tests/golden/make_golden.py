"""Writes tests/golden/reference_vectors.npz: outputs of the reference's own
attention code on seeded synthetic inputs.

The outputs come from oracle/_ref/libnnc_ref.so, which oracle/Makefile
compiles from the reference's libnnc sources (reference src/libnnc/*.cpp,
with the flags of reference CMakeLists.txt:66-76); the layer-level cases
run nnc_attn_block / nnc_attn_merge / nnc_attn_finish (reference
nn_ops.cpp:448-499) through nnc's own worker pool, with the dispatch of
reference model.cpp:1229-1317, 1693-1757 (oracle/ref_driver.cpp). Inputs are
not stored: they are regenerated from the splitmix64 + Box-Muller streams of
libllmcpu_amd.synth, and their SHA-256 is stored so a test notices when the
regeneration drifts.

Run from the repository root, where oracle/_ref is built:
    python3 tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from libllmcpu_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent / "reference_vectors.npz"

# (name, config, layer, n_seq, pos0, n_tok, n_batch, stride): a session that
# appended positions 0 .. n_seq - 1, then attends tokens pos0 .. pos0 + n_tok
# - 1; the output rows of every stride-th token are stored.
LAYER_CASES = [
    ("A_decode", "A", 1, 1024, 1023, 1, 16, 1),            # F32 K/V, hd 256
    ("B_decode", "B", 0, 512, 511, 1, 16, 1),              # hd 64, RoPE NORM
    ("C_local_ring_decode", "C", 0, 3000, 2999, 1, 2048, 1),  # ring of 2560 rows, window 512, wrapped
    ("C_global_prefill", "C", 5, 640, 632, 8, 16, 1),
    ("D_decode", "D", 0, 2048, 2047, 1, 16, 1),            # RMS-normed Q/K, hd 128
    ("D_prefill", "D", 1, 512, 504, 8, 16, 1),
    ("E_local_prefill", "E", 0, 1400, 1392, 8, 1024, 1),  # ring of 2048 rows, window 1024, g = 2
    # chunks long enough for the MFMA prefill kernel: hd 128, and hd 256 on a global layer
    ("D_prefill_chunk64", "D", 1, 2048, 1984, 64, 64, 4),
    ("E_global_chunk64", "E", 5, 1600, 1536, 64, 64, 4),
]


def sha(*arrays: np.ndarray) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_inputs(key: str, layer: int, n_seq: int, pos0: int, n_tok: int, n_batch: int):
    cfg = synth.CONFIGS[key]
    rows = cfg.layer_rows(layer, n_seq, n_batch)
    K, V = synth.cache_buffer(cfg, layer, rows, n_seq)
    q = synth.qk_rows(cfg, layer, 0, np.arange(pos0, pos0 + n_tok), cfg.n_head)
    kw = dict(kv_bf16=cfg.kv_bf16, rows=rows, pos0=pos0, n_seq=n_seq, window=cfg.layer_window(layer), causal=True,
              n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
    return q, K, V, kw


def block_case(orc: oracle.Oracle, lib, which: int):
    """Case `which` of the reference's own block test (tests.cpp:2450-2496):
    3 query heads on KV head 1 of 2, 600 keys in blocks of 100 / 256 / 244."""
    hd, q, K, V = orc.ref_fixture_attn_blocks(which)
    bf16 = which >= 2
    kp, vp = (orc.bf16_round(K), orc.bf16_round(V)) if bf16 else (K, V)
    scale = np.float32(1.0 / np.sqrt(np.float32(hd)))
    acc, k0 = None, 0
    for n in (100, 256, 244):
        kb = np.ascontiguousarray(kp.reshape(-1)[k0 * 2 * hd + hd:])
        vb = np.ascontiguousarray(vp.reshape(-1)[k0 * 2 * hd + hd:])
        part = lib.attn_block(q, kb, vb, bf16, 2 * hd, n, hd, 3, scale)
        acc = part if acc is None else lib.attn_merge(acc, part, hd, 3)
        k0 += n
    return sha(q, kp, vp), lib.attn_finish(acc, hd, 3)


def span_grid():
    rng = np.random.default_rng(20)
    rows = []
    for _ in range(400):
        causal = int(rng.integers(2))
        w = int(rng.choice([0, 1, 3, 40, 512, 1024]))
        n_seq = int(rng.integers(1, 5000))
        pos = int(rng.integers(0, n_seq + 3))
        rows.append((causal, w, pos, n_seq))
    return np.array(rows, dtype=np.int32)


def bf16_inputs():
    rng = np.random.default_rng(21)
    bits = rng.integers(0, 2 ** 32, 1024, dtype=np.uint64).astype(np.uint32)
    special = np.array([0x3F808000, 0x3F818000, 0x3F808001, 0x3F807FFF, 0, 0x80000000, 0x7F7FFFFF, 0xFF7FFFFF,
                        0x00000001, 0x807FFFFF, 0x7F800000, 0xFF800000], dtype=np.uint32)
    x = np.concatenate([special, bits]).view(np.float32)
    return x[np.isfinite(x)]


def main() -> int:
    if not oracle.reference_available():
        print("oracle/_ref is not built (make -C oracle with /root/reference present)", file=sys.stderr)
        return 1
    orc, ref = oracle.Oracle(), oracle.Reference()
    ref.set_threads(8)
    data: dict[str, np.ndarray] = {}
    for name, key, layer, n_seq, pos0, n_tok, n_batch, stride in LAYER_CASES:
        q, K, V, kw = layer_inputs(key, layer, n_seq, pos0, n_tok, n_batch)
        data[f"layer/{name}/out"] = np.ascontiguousarray(ref.attend_layer(q, K, V, **kw)[::stride])
        data[f"layer/{name}/sha256"] = np.array(sha(q, K, V))
        data[f"layer/{name}/case"] = np.array([layer, n_seq, pos0, n_tok, n_batch], dtype=np.int64)
        data[f"layer/{name}/stride"] = np.array(stride, dtype=np.int64)
        data[f"layer/{name}/config"] = np.array(key)
        print(f"{name}: {data[f'layer/{name}/out'].shape}")
    for which in range(4):
        digest, out = block_case(orc, ref, which)
        data[f"blocks/{which}/out"] = out
        data[f"blocks/{which}/sha256"] = np.array(digest)
    grid = span_grid()
    data["span/args"] = grid
    data["span/out"] = np.array([ref.attn_span(bool(c), w, p, n) for c, w, p, n in grid], dtype=np.int32)
    x = bf16_inputs()
    data["bf16/in"] = x
    data["bf16/out"] = ref.bf16_round(x)
    rng = np.random.default_rng(22)
    xr = rng.standard_normal(4 * 128).astype(np.float32)
    data["rope/in"] = xr
    for mode in (0, 1):
        for pos in (7.0, 4095.0):
            data[f"rope/{mode}/{int(pos)}"] = ref.rope(xr, 4, 128, 128, pos, 500000.0, mode)
    data["rmsnorm/out"] = ref.rmsnorm_groups(xr, 128)
    # RoPE with frequency factors (Llama 3 long-context scaling; 1e30 entries
    # switch a pair off, as Gemma 4's proportional RoPE does), partial rotary
    # dims, long positions; RMSNorm with a learned gamma and without gamma.
    ff = np.exp(rng.uniform(0.0, 3.0, 64)).astype(np.float32)
    ff[-8:] = 1e30
    data["rope_ff/factors"] = ff
    for mode in (0, 1):
        for n_rot in (128, 64):
            for pos in (7.0, 32767.0):
                data[f"rope_ff/{mode}/{n_rot}/{int(pos)}"] = ref.rope_ff(xr, 4, 128, n_rot, pos, 1000000.0, mode,
                                                                          ff[: n_rot // 2])
    gamma = rng.uniform(0.5, 1.5, 128).astype(np.float32)
    data["rmsnorm_gamma/gamma"] = gamma
    data["rmsnorm_gamma/out"] = ref.rmsnorm_gamma(xr, 128, gamma)
    x80 = rng.standard_normal(6 * 80).astype(np.float32)
    g80 = rng.uniform(0.5, 1.5, 80).astype(np.float32)
    data["rmsnorm_gamma80/in"] = x80
    data["rmsnorm_gamma80/gamma"] = g80
    data["rmsnorm_gamma80/out"] = ref.rmsnorm_gamma(x80, 80, g80)
    data["rmsnorm_plain80/out"] = ref.rmsnorm_plain(x80, 80)
    # Qwen3.5's output gate: a length that leaves a tail past the runs of
    # eight, gates from -90 to 90 (both saturated ends), and exact zeros.
    yg = rng.standard_normal(1003).astype(np.float32)
    gg = (rng.standard_normal(1003) * 8.0).astype(np.float32)
    gg[:6] = [0.0, 90.0, -90.0, 40.0, -40.0, 0.0]
    data["gate/y"] = yg
    data["gate/g"] = gg
    data["gate/out"] = ref.mul_sigmoid(yg, gg)
    # The weight gemvs: a 72 x 256 matrix (rows not a multiple of 16), three
    # activation vectors, nnc's quantizers and its BF16 / Q8_0 / Q4_S gemvs.
    wg = (rng.standard_normal((72, 256)) * 0.05).astype(np.float32)
    wg[3, :32] = 0.0  # an all-zero block: scale 0
    xg = rng.standard_normal((3, 256)).astype(np.float32)
    data["gemv/w"] = wg
    data["gemv/x"] = xg
    wb = ref.bf16_round(wg)
    data["gemv/bf16/y"] = ref.gemv_bf16(wb, xg)
    q8 = ref.quantize_q8_0(wg)
    data["gemv/q8_0/qs"], data["gemv/q8_0/scales"] = q8
    data["gemv/q8_0/y"] = ref.gemv_q8_0(*q8, xg)
    q4 = ref.quantize_q4_s(wg)
    data["gemv/q4_s/qs"], data["gemv/q4_s/scales"], data["gemv/q4_s/biases"] = q4
    data["gemv/xsum"] = ref.block_sums(xg)
    data["gemv/q4_s/y"] = ref.gemv_q4_s(*q4, xg)
    # The lm_head argmax: uniform(-1, 1) weights and x as in the reference's
    # own test, on its fast path (rows % 4 == 0, cols % 8 == 0: 64 x 256, with
    # the best row duplicated later, so the first copy must win) and its
    # fallback (7 x 40).
    for name, (rows, cols) in (("fast", (64, 256)), ("fallback", (7, 40))):
        wa = ref.bf16_round(rng.uniform(-1.0, 1.0, (rows, cols)).astype(np.float32))
        xa = rng.uniform(-1.0, 1.0, cols).astype(np.float32)
        if name == "fast":
            top = ref.gemv_bf16_argmax(wa, xa)
            wa[rows - 3 if top != rows - 3 else rows - 1] = wa[top]  # a tie with the best row
        data[f"argmax/{name}/w"] = wa
        data[f"argmax/{name}/x"] = xa
        data[f"argmax/{name}/index"] = np.int32(ref.gemv_bf16_argmax(wa, xa))
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())

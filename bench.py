"""Benchmark of nnc's attention hot path on one MI355X, at the Qwen3-4B shape
(32 query heads, 8 KV heads, head_dim 128, 36 layers, BF16 K/V).

A decode step is one query token through the attention of all 36 layers at
32768 cached positions, each layer reading its own K/V buffer (36 x 128 MiB,
so the working set is far past the 256 MB Infinity Cache). A prefill step is
a 4096-token prompt through all 36 layers in 512-token chunks (8 calls per
layer, chunk c attending to keys 0 .. 512c + 511). Inputs are synthetic and
resident in HBM before timing: K/V/Q ~ N(0,1) from the splitmix64 +
Box-Muller generator, Q and K RMS-normalised per head as Qwen3 does.

Prints one JSON line. `value` is decode K/V bytes per second (the algorithmic
2 * S * n_kv * head_dim * 2 + 2 * n_head * head_dim * 4 bytes per layer);
prefill TFLOP/s (4 * head_dim * n_head * sum of span lengths) rides in
`prefill`. `roofline` is the decode kernel's (HBM bound),
`prefill.roofline` the prefill kernel's (MFMA bound, dense fp16/bf16 peak),
both from HIP events on the op's stream; their `traffic` comes from the
counter summaries in profiles/. Beside them: chunk 7 of the prompt in exact
mode (every token with its one-token bits) against the prefill kernel, a
16-token session batch, the pre-attention step, the weight gemvs, one decode
layer through the host-buffer entry point (C-side cost beside the device
form), the other benchmark configurations (A, B, C, D at 4096 keys, E; each
step replayed from a HIP graph) and `cpu_baseline`, nnc's own CPU attention
(oracle/_ref: the reference's kernels and worker pool) on bounded samples of
the same work on this host (decode at the reference's two thread settings,
a prefill chunk, B at 16384 keys, C's decode step), whose leg also gives the
`parity` block: max-abs and max-rel (|d| / (1 + |ref|)) of the timed GPU
outputs against the reference on the same inputs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

METRIC = json.loads((ROOT / "BASELINE.json").read_text())["metric"]
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16
FP32_MFMA_PEAK_TFLOPS = 157.3  # dense fp32 (the tiled kernel's products on F32 K/V)
ATTR_CU, ATTR_CLOCK = 63, 5  # hipDeviceAttributeMultiprocessorCount, hipDeviceAttributeClockRate

N_HEAD, N_KV, HD, N_LAYER = 32, 8, 128, 36
KV_DIM = N_KV * HD
CTX = 32768
PROMPT, CHUNK = 4096, 512
SESSION_BATCH = 16  # nnc's tokens per forward pass in a session (reference model.h:330)
SCALE = 1.0 / np.sqrt(HD)


def decode_bytes(span: int) -> int:
    return 2 * span * KV_DIM * 2 + 2 * N_HEAD * HD * 4


def prep_bytes(n_tok: int) -> int:
    """Algorithmic bytes of the pre-attention step of one layer (reference
    model.cpp:1616-1691): q read and written, k and v read (fp32), the K and V
    rows written (BF16), the two gammas read."""
    return n_tok * (N_HEAD * HD * 4 * 2 + KV_DIM * 4 * 2 + KV_DIM * 2 * 2) + 2 * HD * 4


def prefill_flops(pos0: int, n_tok: int) -> int:
    spans = np.arange(pos0 + 1, pos0 + n_tok + 1, dtype=np.int64)  # causal: key 0 .. pos
    return int(4 * HD * N_HEAD * spans.sum())


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


BOX_CPU_SHARE = 16  # host CPUs one GPU's jobs may use on the GPU boxes


def cpu_model() -> str:
    """/proc/cpuinfo's model name with its family, model and stepping (a VM
    may report only "AMD EPYC"; family 26 is AMD's Zen 5 generation)."""
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("model name", "cpu family", "model", "stepping", "flags") and k not in info:
                info[k] = v.strip()
            if len(info) == 5:
                break
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    extra = ", ".join(f"{k} {info[k]}" for k in ("cpu family", "model", "stepping") if k in info)
    flags = info.get("flags", "").split()
    tags = [t for t in ("avx512f", "avx512_bf16", "hypervisor") if t in flags]
    return f"{name} ({extra}{'; ' + ' '.join(tags) if tags else ''})" if extra else name


def parity_of(got: np.ndarray, ref: np.ndarray) -> dict:
    """max-abs and max-rel, rel = |d| / (1 + |ref|), of the GPU output against the reference's."""
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return {"max_abs": float(d.max()), "max_rel": float((d / (1.0 + np.abs(ref))).max())}


def cpu_baseline(cache_l0, target_s: float, samples: dict) -> dict:
    """nnc's CPU attention on this host (oracle/_ref: the reference's own
    kernels and worker pool, or the oracle's port where it was not built),
    on bounded samples of the benchmark's work, and the parity of the timed
    GPU outputs against it on the same inputs.

    Decode: one Qwen3-4B layer at 32768 keys (layer 0 of the timed step: its
    q and the GPU's output), repeated for about target_s seconds per setting,
    at the reference's two thread settings: min(8, nproc) (its default,
    reference nn_ops.cpp:865-879) and nproc capped at 64 (nn_ops.cpp:786),
    the latter also held to the CPUs this process may use. The first is the
    reported value. Prefill: chunk 7 of layer 0 (512 tokens at keys 0 ..
    4095), the GPU's output of the same call. B decode at 16384 keys, C's
    26-layer decode step at 8192 (22 windowed local layers, 4 global), A's
    F32 decode step and E's decode step after its prompt, on synthetic rows
    of their shapes, at the default setting."""
    import oracle

    K, V = cache_l0
    nproc = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else nproc
    ref = oracle.reference_available()
    lib = oracle.Reference() if ref else oracle.Oracle()
    kind = "reference" if ref else "port"

    def attend(threads, q, Kb, Vb, **kw):
        if ref:
            lib.set_threads(threads)
            return lib.attend_layer(q, Kb, Vb, **kw)
        return lib.attend_layer(q, Kb, Vb, threads=threads, **kw)

    def best_of(threads, seconds, q, Kb, Vb, **kw):
        out = attend(threads, q, Kb, Vb, **kw)
        n, t0, best = 0, time.perf_counter(), float("inf")
        while n < 2 or time.perf_counter() - t0 < seconds:
            t = time.perf_counter()
            attend(threads, q, Kb, Vb, **kw)
            best = min(best, time.perf_counter() - t)
            n += 1
        return out, best, n

    t_default = min(8, nproc)
    t_all = min(64, nproc, usable, BOX_CPU_SHARE)
    dec = dict(kv_bf16=True, rows=CTX, pos0=CTX - 1, n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)
    q0 = samples["decode_q"]
    ref_dec, best, n = best_of(t_default, target_s, q0, K, V, **dec)
    _, best_all, n_all = best_of(t_all, target_s, q0, K, V, **dec)
    gbs, gbs_all = decode_bytes(CTX) / best / 1e9, decode_bytes(CTX) / best_all / 1e9

    # prefill: chunk 7 of layer 0
    c0 = (PROMPT // CHUNK - 1) * CHUNK
    pre = dict(kv_bf16=True, rows=PROMPT, pos0=c0, n_seq=c0 + CHUNK, n_head=N_HEAD, n_kv=N_KV, head_dim=HD,
               scale=SCALE)
    ref_pre, best_pre, n_pre = best_of(t_default, 2.0, samples["prefill_q"], K[:PROMPT], V[:PROMPT], **pre)
    pre_tflops = prefill_flops(c0, CHUNK) / best_pre / 1e12

    # B decode at 16384 keys and C's decode step, on synthetic rows of their shapes
    from libllmcpu_amd import synth
    rng = np.random.default_rng(5)

    def decode_layer_s(cfg, rows, window, span_keys):
        Kb = rng.standard_normal((rows, cfg.kv_dim)).astype(np.float32)
        Vb = rng.standard_normal((rows, cfg.kv_dim)).astype(np.float32)
        if cfg.kv_bf16:
            Kb, Vb = nh_bf16(Kb), nh_bf16(Vb)
        q = rng.standard_normal((1, cfg.n_head * cfg.head_dim)).astype(np.float32)
        kw = dict(kv_bf16=cfg.kv_bf16, rows=rows, pos0=span_keys - 1, n_seq=span_keys, window=window,
                  n_head=cfg.n_head, n_kv=cfg.n_kv, head_dim=cfg.head_dim, scale=cfg.attn_scale)
        return best_of(t_default, 1.0, q, Kb, Vb, **kw)[1]

    B, Cc = synth.CONFIGS["B"], synth.CONFIGS["C"]
    b_s = decode_layer_s(B, 16384, 0, 16384)
    b_bytes = decode_layer_bytes(16384, B.n_kv, B.head_dim, B.n_head, 2)
    n_local = sum(1 for li in range(Cc.n_layer) if Cc.layer_window(li) > 0)
    c_local = decode_layer_s(Cc, Cc.layer_rows(0, 8192, 2048), Cc.window, 8192)
    c_global = decode_layer_s(Cc, 8192, 0, 8192)
    c_step = n_local * c_local + (Cc.n_layer - n_local) * c_global
    c_bytes = sum(decode_layer_bytes(int(layer_spans(Cc, li, 8191, 1)[0]), Cc.n_kv, Cc.head_dim, Cc.n_head, 2)
                  for li in range(Cc.n_layer))
    # A's decode step (F32, 18 layers at 1024 keys) and one of E's 256 decode
    # steps after the 16384-token prompt (at position 16511, the middle one)
    A, E = synth.CONFIGS["A"], synth.CONFIGS["E"]
    a_step = A.n_layer * decode_layer_s(A, 1024, 0, 1024)
    a_bytes = A.n_layer * decode_layer_bytes(1024, A.n_kv, A.head_dim, A.n_head, 4)
    e_pos, e_ctx = 16511, 16384 + 256
    e_local_n = sum(1 for li in range(E.n_layer) if E.layer_window(li) > 0)
    e_local = decode_layer_s(E, E.layer_rows(0, e_ctx, 1024), E.window, e_pos + 1)
    e_global = decode_layer_s(E, e_ctx, 0, e_pos + 1)
    e_step = e_local_n * e_local + (E.n_layer - e_local_n) * e_global
    e_bytes = sum(decode_layer_bytes(int(layer_spans(E, li, e_pos, 1)[0]), E.n_kv, E.head_dim, E.n_head, 2)
                  for li in range(E.n_layer))
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": t_default, "kind": kind,
            "sample": f"decode of one Qwen3-4B layer at {CTX} keys (layer 0 of the timed step), best of {n} runs "
                      f"over {target_s:.0f} s (the reference's kernels and worker pool)",
            "cpu": cpu_model(), "nproc": nproc, "usable_cpus": usable,
            "all_cores": {"value": round(gbs_all, 2), "cores": t_all, "runs": n_all,
                          "threads_rule": f"min(64, nproc) held to the usable CPUs and the box's "
                                          f"{BOX_CPU_SHARE}-CPU share per GPU"},
            "prefill": {"value": round(pre_tflops, 4), "unit": "TFLOP/s", "cores": t_default, "runs": n_pre,
                        "sample": f"chunk 7 of layer 0 (512 tokens at keys 0 .. 4095), {best_pre * 1e3:.1f} ms"},
            "B_decode_16384": {"value": round(b_bytes / b_s / 1e9, 2), "unit": "GB/s", "cores": t_default,
                               "sample": "one Llama-3.2-1B layer at 16384 keys, synthetic rows"},
            "C_decode_8192": {"value": round(c_bytes / c_step / 1e9, 2), "unit": "GB/s", "cores": t_default,
                              "ms_per_step": round(c_step * 1e3, 3),
                              "sample": f"{n_local} local (window {Cc.window}) and {Cc.n_layer - n_local} global "
                                        f"Gemma-3-1B layers at 8192, synthetic rows"},
            "A_decode_1024": {"value": round(a_bytes / a_step / 1e9, 2), "unit": "GB/s", "cores": t_default,
                              "ms_per_step": round(a_step * 1e3, 3),
                              "sample": "18 Gemma-3-270M layers (F32 K/V) at 1024 keys, synthetic rows"},
            "E_decode_256": {"value": round(e_bytes / e_step / 1e9, 2), "unit": "GB/s", "cores": t_default,
                             "ms_per_step": round(e_step * 1e3, 3),
                             "sample": f"the decode step at position {e_pos}: {e_local_n} local (window {E.window}) and "
                                       f"{E.n_layer - e_local_n} global Gemma-3-4B layers, synthetic rows"},
            "parity": {"against": kind, "rel": "|d| / (1 + |ref|)",
                       "decode_layer0_32768": parity_of(samples["decode_out"], ref_dec),
                       "prefill_layer0_chunk7": parity_of(samples["prefill_out"], ref_pre),
                       "bound": 5e-3}}


def nh_bf16(x: np.ndarray) -> np.ndarray:
    from libllmcpu_amd import bf16_round
    return bf16_round(x)


def pmc_summary(fetch_csv: str, write_csv: str, kind: str = "decode") -> dict:
    """HBM bytes per attend call from two `rocprofv3 --pmc` runs of
    `bench.py --only decode|prefill --calibrate` (FETCH_SIZE, then WRITE_SIZE,
    both in KiB per dispatch). The copy of CALIBRATE_MIB MiB that such a run
    starts with reads and writes exactly that many bytes, which converts each
    counter to bytes. decode: one call is decode_bf16_kernel +
    decode_merge_kernel at 32768 keys; prefill: one call is one
    prefill_kernel launch, averaged over the 8 chunks of the 4096-token
    prompt (chunk c reads keys 0 .. 512 c + 511)."""
    import csv

    def per_kernel(path):
        acc = {}
        for r in csv.DictReader(open(path)):
            name = r["Kernel_Name"]
            key = ("copy" if "copy" in name.lower() else "merge" if "decode_merge" in name
                   else "decode" if "decode" in name else "prefill" if "prefill" in name else None)
            if key:
                acc.setdefault(key, []).append(float(r["Counter_Value"]))
        return {k: float(np.median(v) if k != "prefill" else np.mean(v)) for k, v in acc.items()}

    f, w = per_kernel(fetch_csv), per_kernel(write_csv)
    copy_bytes = CALIBRATE_MIB << 20
    f_scale = copy_bytes / (f["copy"] * 1024)
    w_scale = copy_bytes / (w["copy"] * 1024)
    parts = ("decode", "merge") if kind == "decode" else ("prefill",)
    fetch = sum(f.get(k, 0.0) for k in parts) * 1024 * f_scale
    write = sum(w.get(k, 0.0) for k in parts) * 1024 * w_scale
    out = {"hbm_bytes_per_launch": int(round(fetch + write)), "fetch_bytes": int(round(fetch)),
           "write_bytes": int(round(write)),
           "fetch_kib_per_dispatch": {k: round(v, 1) for k, v in f.items()},
           "write_kib_per_dispatch": {k: round(v, 1) for k, v in w.items()},
           "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
           "calibration": f"torch copy_ of {CALIBRATE_MIB} MiB (reads and writes {copy_bytes} bytes)"}
    if kind == "decode":
        out.update(algorithmic_bytes=decode_bytes(CTX), launch="one attend call: decode_bf16_kernel + decode_merge_kernel")
    else:
        kv_bytes = np.mean([2 * (c + 1) * CHUNK * KV_DIM * 2 for c in range(PROMPT // CHUNK)])
        out.update(kv_bytes_per_launch=int(kv_bytes), q_out_bytes_per_launch=2 * CHUNK * N_HEAD * HD * 4,
                   launch="one prefill_kernel launch (a 512-token chunk), mean over the 8 chunks")
    return out


def counter_summary(paths: list, pattern: str, clock_mhz: float = 2400.0) -> dict:
    """Per-dispatch counter values of the kernels whose name contains
    `pattern`, from `rocprofv3 --pmc ... --output-format csv` files, averaged
    over dispatches (a counter listed twice for one dispatch is counted once),
    and busy fractions over the dispatch's duration (its timestamps) at
    clock_mhz: SQ_VALU_MFMA_BUSY_CYCLES over the 1024 SIMDs (matrix cores
    busy), SQ_VALU_MFMA_COEXEC_CYCLES (matrix core and vector ALU busy at
    once), TA_BUSY_avr (the texture-address units that issue the loads)."""
    import csv

    per, dur = {}, {}
    for path in paths:
        for r in csv.DictReader(open(path)):
            if pattern not in r["Kernel_Name"]:
                continue
            d = int(r["Dispatch_Id"])
            per.setdefault(r["Counter_Name"], {})[d] = float(r["Counter_Value"])
            dur[d] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
    mean = {k: float(np.mean(list(v.values()))) for k, v in per.items()}
    out = {"dispatches": max(len(v) for v in per.values()) if per else 0,
           "mean_per_dispatch": {k: round(v, 1) for k, v in sorted(mean.items())}}
    if dur:
        cycles = float(np.mean(list(dur.values()))) * clock_mhz * 1e6
        out["mean_duration_us"] = round(float(np.mean(list(dur.values()))) * 1e6, 3)
        out["clock_mhz"] = clock_mhz
        simds = 4 * 256
        if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
            out["mfma_busy"] = round(mean["SQ_VALU_MFMA_BUSY_CYCLES"] / (simds * cycles), 4)
        if "SQ_VALU_MFMA_COEXEC_CYCLES" in mean:
            out["mfma_valu_coexec"] = round(mean["SQ_VALU_MFMA_COEXEC_CYCLES"] / (simds * cycles), 4)
        if "TA_BUSY_avr" in mean:
            out["ta_busy"] = round(mean["TA_BUSY_avr"] / cycles, 4)
    return out


CALIBRATE_MIB = 1024


# Qwen3-4B's weight gemvs of one layer (rows, cols): q, k, v, o, gate, up, down.
GEMV_LAYER = [(4096, 2560), (1024, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (9728, 2560), (2560, 9728)]
GEMV_GROUPS = [(0, 1, 2), (3,), (4, 5), (6,)]  # launches per layer: q/k/v and gate/up share their input
LM_HEAD = (151936, 2560)  # Qwen3-4B vocabulary x n_embd
GEMV_WORKING_SET = 640 << 20  # bytes of distinct weights per format, past the 256 MB Infinity Cache


def gemv_bytes(fmt: str, rows: int, cols: int) -> int:
    """Weight bytes of one matrix in nnc's layouts (reference docs/design.md:141-193)."""
    return {"bf16": 2 * rows * cols, "q8_0": rows * cols + 2 * rows * cols // 32,
            "q4_s": rows * cols // 2 + 4 * rows * cols // 32}[fmt]


def gemv_bench(nh, hip_rt, kv, stream, timed) -> dict:
    """The weight gemvs of Qwen3-4B layers in each of nnc's three weight
    layouts, one activation vector (decode) and 16 (a session batch), weights
    resident in HBM and rotated over enough layers to exceed the Infinity
    Cache. Algorithmic bytes: the weights (with scales and biases) plus X and Y."""
    res = {}
    x = hip_rt.malloc(16 * 9728 * 4)
    y = hip_rt.malloc(16 * 2 * 9728 * 4)  # room for a group's outputs side by side
    nh.fill_normal(x, 16 * 9728, 99, 0, False, stream)
    # Every buffer is freed only after the last timing: the driver clears freed
    # device memory in the background, which takes HBM bandwidth for seconds.
    bufs = []
    for fmt in ("bf16", "q8_0", "q4_s"):
        layer_bytes = sum(gemv_bytes(fmt, r, c) for r, c in GEMV_LAYER)
        n_layers = -(-GEMV_WORKING_SET // layer_bytes)
        mats = []
        for li in range(n_layers):
            for mi, (r, c) in enumerate(GEMV_LAYER):
                parts = {"bf16": [2 * r * c], "q8_0": [r * c, 2 * r * c // 32],
                         "q4_s": [r * c // 2, 2 * r * c // 32, 2 * r * c // 32]}[fmt]
                ptrs = []
                for j, nbytes in enumerate(parts):
                    d = hip_rt.malloc(nbytes)
                    # Random bits: BF16 N(0,1) pairs (weights, scales, or int8 / nibble bytes).
                    nh.fill_normal(d, nbytes // 2, 5000 + 100 * li + 10 * mi + j, 0, True, stream)
                    bufs.append(d)
                    ptrs.append(d)
                mats.append((tuple(ptrs), r, c))
        kv.sync()
        for n in (1, 16):
            def step():
                # Per layer: q, k and v over the same input in one launch, then
                # o, gate and up (one launch), down.
                for li in range(0, len(mats), len(GEMV_LAYER)):
                    lm = mats[li:li + len(GEMV_LAYER)]
                    for grp in GEMV_GROUPS:
                        if len(grp) == 1:
                            w, r, c = lm[grp[0]]
                            kv.gemv_device(fmt, w, x, y, rows=r, cols=c, n_batch=n)
                        else:
                            ys = [y + 4 * 16 * sum(lm[j][1] for j in grp[:k]) for k in range(len(grp))]
                            kv.gemv_group_device(fmt, [(lm[j][0], ys[k], lm[j][1]) for k, j in enumerate(grp)], x,
                                                 cols=lm[grp[0]][2], n_batch=n)

            step()
            hip_rt.sync()
            ms, _ = timed(step, 5)
            us_layer = ms * 1e3 / (5 * n_layers)
            nbytes = layer_bytes + sum(4 * n * (r + c) for r, c in GEMV_LAYER)
            gbs = nbytes / (us_layer * 1e-6) / 1e9
            res[f"{fmt}_n{n}"] = {"us_per_layer": round(us_layer, 2), "bytes_per_layer": nbytes,
                                  "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # Greedy decode's lm_head: the argmax of the BF16 projection onto the
    # vocabulary (Qwen3-4B ties it to the token embeddings), 778 MB per call;
    # the call waits for its result, so the time includes the index's copy
    # back and the host's return.
    rows, cols = LM_HEAD
    w = hip_rt.malloc(2 * rows * cols)
    nh.fill_normal(w, rows * cols, 7777, 0, True, stream)
    kv.sync()
    kv.gemv_argmax_device(w, x, rows=rows, cols=cols)
    n_calls = 10
    _, wall_ms = timed(lambda: kv.gemv_argmax_device(w, x, rows=rows, cols=cols), n_calls)
    us = wall_ms * 1e3 / n_calls
    nbytes = 2 * rows * cols + 4 * cols
    res["lm_head_argmax"] = {"rows": rows, "cols": cols, "us_per_call": round(us, 2), "bytes": nbytes,
                             "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
                             "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                             "kernels": "gemv_vec_kernel<bf16, argmax> + gemv_argmax_final_kernel"}
    for d in bufs + [w, x, y]:
        hip_rt.free(d)
    return {"what": "Qwen3-4B layer weight gemvs (q, k, v, o, gate, up, down) per weight layout; n1 = one "
                    "vector (decode), n16 = a 16-token session batch; weights in HBM, rotated past the "
                    "Infinity Cache; four launches per layer (q/k/v and gate/up as nnc_hip_gemv_group calls)", "bound": "hbm", "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "kernels": "gemv_vec_kernel (one vector), gemv_kernel + gemv_reduce_kernel (batches)", **res}


def decode_layer_bytes(span: int, n_kv: int, hd: int, n_head: int, esize: int) -> int:
    """Algorithmic bytes of one decode call: K and V over the span, q in and out."""
    return 2 * span * n_kv * hd * esize + 2 * n_head * hd * 4


def layer_spans(cfg, layer: int, pos0: int, n_tok: int) -> np.ndarray:
    """Keys each query of a causal batch sees (a window caps local layers)."""
    pos = np.arange(pos0, pos0 + n_tok, dtype=np.int64)
    w = cfg.layer_window(layer)
    return np.minimum(pos + 1, w) if w > 0 else pos + 1


def configs_bench(nh, hip_rt, synth) -> dict:
    """The benchmark's other configurations (A, B, C, D at 4096, E) and an
    embedding call (EmbeddingGemma-300M's shape), each
    step replayed from a HIP graph of its attend calls so the small layers are
    timed by the GPU rather than by Python's launch rate. Inputs come from
    the device generator (K RMS-normed per head where the model normalises
    it); every layer's buffer holds the positions the step reads (a sliding
    layer's ring the last `rows` of them). A replay is checked bit for bit
    against an eager run of the same calls. Algorithmic work per the
    decode-bytes and prefill-flops formulas of the headline line."""
    import ctypes as C

    lib = nh.load_library()
    out = {}
    # Caches and fill buffers live until the end: nothing is freed before a
    # timed step (the driver clears freed device memory in the background).
    keep = []

    def build(cfg, n_ctx, n_batch):
        rows = [cfg.layer_rows(li, n_ctx, n_batch) for li in range(cfg.n_layer)]
        kv = nh.KVCache(rows, [cfg.kv_dim] * cfg.n_layer, bf16=cfg.kv_bf16)
        st = kv.stream
        n_max = max(rows) * cfg.kv_dim
        k_dev, v_dev = hip_rt.malloc(4 * n_max), hip_rt.malloc(4 * n_max)
        keep.append((kv, k_dev, v_dev))
        for li, r in enumerate(rows):
            seed = (synth.BASE_SEED + 1000 * cfg.index + li) * 256
            nh.fill_normal(k_dev, r * cfg.kv_dim, seed + 1, cfg.head_dim if cfg.qk_norm else 0, False, st)
            nh.fill_normal(v_dev, r * cfg.kv_dim, seed + 2, 0, False, st)
            first = n_ctx - r  # the ring keeps the newest rows
            status = lib.nnc_hip_kv_append_f32_device(kv.handle, li, first, r, C.c_void_p(k_dev), C.c_void_p(v_dev))
            if status:
                raise nh.NncError(status, lib.nnc_hip_last_error().decode())
        kv.sync()
        return kv

    def measure(kv, calls, n_tok_max, n_out, cfg, reps, causal=True):
        """calls: (layer, out slot, pos0, n_tok) tuples of one step."""
        st = kv.stream
        width = cfg.n_head * cfg.head_dim
        q = hip_rt.malloc(4 * n_tok_max * width)
        o = hip_rt.malloc(4 * n_out * n_tok_max * width)
        nh.fill_normal(q, n_tok_max * width, 4242 + cfg.index, cfg.head_dim if cfg.qk_norm else 0, False, st)

        def step():
            for li, slot, pos0, n in calls:
                kv.attend_device(li, q, o + 4 * slot * n_tok_max * width, n_tok=n, pos0=pos0,
                                 window=cfg.layer_window(li), causal=causal, n_head=cfg.n_head, n_kv=cfg.n_kv,
                                 head_dim=cfg.head_dim, scale=cfg.attn_scale)

        step()  # eager: scratch grows here, never inside the capture
        kv.sync()
        eager = hip_rt.to_host(np.empty(n_out * n_tok_max * width, np.float32), o)
        graph = hip_rt.Graph(st, step)
        graph.launch(st)
        kv.sync()
        e0, e1 = hip_rt.Event(), hip_rt.Event()
        e0.record(st)
        for _ in range(reps):
            graph.launch(st)
        e1.record(st)
        e1.synchronize()
        ms = e1.ms_since(e0) / reps
        replay = hip_rt.to_host(np.empty_like(eager), o)
        graph.close()
        same = bool(np.array_equal(eager.view(np.uint32), replay.view(np.uint32)))
        hip_rt.free(q)
        hip_rt.free(o)
        return ms, same

    def decode_entry(cfg, label, kv, ctx, reps=20):
        calls = [(li, li, ctx - 1, 1) for li in range(cfg.n_layer)]
        ms, same = measure(kv, calls, 1, cfg.n_layer, cfg, reps)
        esize = 2 if cfg.kv_bf16 else 4
        nbytes = sum(decode_layer_bytes(int(layer_spans(cfg, li, ctx - 1, 1)[0]), cfg.n_kv, cfg.head_dim, cfg.n_head,
                                        esize) for li in range(cfg.n_layer))
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[label] = {"workload": f"{cfg.name}: one decode token at {ctx} keys through {cfg.n_layer} layers",
                      "ms_per_step": round(ms, 4), "bytes_per_step": nbytes, "value": round(gbs, 1), "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4), "replay_equals_eager": same}
        log(f"[bench] {label}: {ms * 1e3:.1f} us/step, {gbs:.0f} GB/s")

    def prefill_entry(cfg, label, kv, n_prompt, chunk, reps=3):
        calls = [(li, c, c * chunk, chunk) for li in range(cfg.n_layer) for c in range(n_prompt // chunk)]
        ms, same = measure(kv, calls, chunk, n_prompt // chunk, cfg, reps)
        flops = sum(int(4 * cfg.head_dim * cfg.n_head * layer_spans(cfg, li, 0, n_prompt).sum())
                    for li in range(cfg.n_layer))
        tf = flops / (ms * 1e-3) / 1e12
        out[label] = {"workload": f"{cfg.name}: a {n_prompt}-token prompt in {chunk}-token chunks through "
                                  f"{cfg.n_layer} layers", "ms_per_step": round(ms, 3), "flops_per_step": flops,
                      "value": round(tf, 1), "unit": "TFLOP/s", "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
                      "replay_equals_eager": same}
        log(f"[bench] {label}: {ms:.3f} ms/step, {tf:.0f} TFLOP/s")

    A, B, Cc, D, E = (synth.CONFIGS[k] for k in "ABCDE")
    kv = build(A, 1024, 1)
    decode_entry(A, "A_decode_1024", kv, 1024, reps=50)
    out["A_decode_1024"]["note"] = "18 x 2 MB of K/V stay in the 256 MB Infinity Cache: not an HBM rate"
    kv = build(B, 16384, 1)
    for ctx in (512, 4096, 16384):
        decode_entry(B, f"B_decode_{ctx}", kv, ctx)
    kv = build(D, 4096, 1)
    decode_entry(D, "D_decode_4096", kv, 4096)
    kv = build(Cc, 8192, 2048)
    decode_entry(Cc, "C_decode_8192", kv, 8192)
    prefill_entry(Cc, "C_prefill_8192", kv, 8192, 2048)
    n_ctx = 16384 + 256
    kv = build(E, n_ctx, 1024)
    prefill_entry(E, "E_prefill_16384", kv, 16384, 1024, reps=2)
    # 256 decode steps after the prompt, one graph
    calls = [(li, li, p, 1) for p in range(16384, n_ctx) for li in range(E.n_layer)]
    ms, same = measure(kv, calls, 1, E.n_layer, E, 2)
    nbytes = sum(decode_layer_bytes(int(layer_spans(E, li, p, 1)[0]), E.n_kv, E.head_dim, E.n_head, 2)
                 for p in range(16384, n_ctx) for li in range(E.n_layer))
    gbs = nbytes / (ms * 1e-3) / 1e9
    out["E_decode_256"] = {"workload": f"{E.name}: 256 decode steps after a 16384-token prompt, {E.n_layer} layers",
                           "ms_per_step": round(ms / 256, 4), "bytes_per_step": nbytes // 256, "value": round(gbs, 1),
                           "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "replay_equals_eager": same}
    log(f"[bench] E_decode_256: {ms / 256 * 1e3:.1f} us/step, {gbs:.0f} GB/s")
    # nnc's embedding call (reference model.cpp:2355-2368): the whole input
    # in one batch over an F32 cache, bidirectional (local layers see +-w/2
    # keys, model.cpp:2308-2315), EmbeddingGemma-300M's attention shape.
    emb = synth.AttnConfig(5, "embeddinggemma-300m embedding", 3, 1, 256, 24, kv_bf16=False, window=512,
                           swa_period=6, tol=1e-3)
    n_emb = 2048
    kv = build(emb, n_emb, n_emb)
    calls = [(li, li, 0, n_emb) for li in range(emb.n_layer)]
    ms, same = measure(kv, calls, n_emb, emb.n_layer, emb, 3, causal=False)
    pos = np.arange(n_emb, dtype=np.int64)
    flops = 0
    for li in range(emb.n_layer):
        w = emb.layer_window(li)
        spans = (np.minimum(n_emb - 1, pos + w // 2) - np.maximum(0, pos - w // 2) + 1) if w > 0 else \
            np.full(n_emb, n_emb)
        flops += int(4 * emb.head_dim * emb.n_head * spans.sum())
    tf = flops / (ms * 1e-3) / 1e12
    out["EMB_embed_2048"] = {"workload": f"{emb.name}: one {n_emb}-token input, F32 K/V, bidirectional, "
                                         f"{emb.n_layer} layers (20 with a 512-key window)",
                             "ms_per_step": round(ms, 3), "flops_per_step": flops, "value": round(tf, 2),
                             "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
                             "peak": "fp32 MFMA, 157.3 TFLOP/s", "replay_equals_eager": same}
    log(f"[bench] EMB_embed_2048: {ms:.3f} ms/step, {tf:.1f} TFLOP/s")
    for kv_, k_dev, v_dev in keep:
        kv_.close()
        hip_rt.free(k_dev)
        hip_rt.free(v_dev)
    return out


def host_path_bench(nh, kv, q_dev: int, o_dev: int) -> dict:
    """One decode layer through nnc_hip_attend (q and out in host memory, the
    call synchronous), as a drop-in caller at reference model.cpp:1693-1757
    would make it, beside the device form made synchronous
    (nnc_hip_attend_device + nnc_hip_kv_sync). Both through raw ctypes calls;
    the C-side cost per call is the wall time less the cost of a ctypes call
    that returns at once (nnc_hip_kv_bytes), measured the same way."""
    import ctypes as C

    lib = nh.load_library()
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, N_HEAD * HD)).astype(np.float32)
    out = np.empty_like(q)
    qp, op, h = C.c_void_p(q.ctypes.data), C.c_void_p(out.ctypes.data), kv.handle
    args = (1, CTX - 1, CTX, 0, True, N_HEAD, N_KV, HD, SCALE)
    reps = 5

    def per_call(fn):
        fn()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        return (time.perf_counter() - t0) * 1e6 / (reps * N_LAYER)

    def host():
        for li in range(N_LAYER):
            lib.nnc_hip_attend(h, li, qp, op, *args)

    def device():
        for li in range(N_LAYER):
            lib.nnc_hip_attend_device(h, li, C.c_void_p(q_dev + li * N_HEAD * HD * 4),
                                      C.c_void_p(o_dev + li * N_HEAD * HD * 4), *args)
            lib.nnc_hip_kv_sync(h)

    def floor():
        for _ in range(N_LAYER):
            lib.nnc_hip_kv_bytes(h)

    host_us, dev_us, floor_us = per_call(host), per_call(device), per_call(floor)
    c_host, c_dev = host_us - floor_us, dev_us - 2 * floor_us
    return {"what": "one Qwen3-4B decode layer at 32768 keys through nnc_hip_attend: q copied into pinned memory "
                    "and read by a copy kernel, out written by the kernels into pinned memory, the call "
                    "synchronous; beside nnc_hip_attend_device + nnc_hip_kv_sync on the same layers",
            "us_per_call": round(host_us, 2), "c_side_us": round(c_host, 2),
            "device_form_c_side_us": round(c_dev, 2), "ratio_to_device_form": round(c_host / c_dev, 3),
            "ctypes_call_us": round(floor_us, 3),
            "gbs": round(decode_bytes(CTX) / (c_host * 1e-6) / 1e9, 1)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--prefill-steps", type=int, default=3)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other configurations (A, B, C, D at 4096, E)")
    ap.add_argument("--only", choices=["decode", "prefill", "batch", "prep", "gemv", "configs"], default=None,
                    help="time one mode only (profiling runs); the JSON line needs both")
    ap.add_argument("--traffic", default=str(ROOT / "profiles" / "decode_traffic.json"),
                    help="rocprofv3 --pmc summary giving HBM bytes per decode launch")
    ap.add_argument("--prefill-traffic", default=str(ROOT / "profiles" / "prefill_counters.json"),
                    help="rocprofv3 --pmc summary giving HBM bytes per prefill launch")
    ap.add_argument("--calibrate", action="store_true",
                    help=f"start with a {CALIBRATE_MIB} MiB copy kernel (counter calibration)")
    ap.add_argument("--pmc-summary", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="print the HBM traffic summary of two rocprofv3 --pmc runs and exit (no GPU)")
    ap.add_argument("--pmc-kind", choices=["decode", "prefill"], default="decode",
                    help="which attend call --pmc-summary describes")
    ap.add_argument("--counter-summary", nargs="+", metavar="CSV",
                    help="print per-dispatch averages and busy fractions of rocprofv3 --pmc runs and exit (no GPU)")
    ap.add_argument("--kernel", default="prefill_kernel", help="kernel name pattern for --counter-summary")
    args = ap.parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_summary(*args.pmc_summary, kind=args.pmc_kind), indent=1))
        return 0
    if args.counter_summary:
        print(json.dumps(counter_summary(args.counter_summary, args.kernel), indent=1))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (this build has no "
              "multi-GPU path; the op would shard by KV head, or by key range with one exchange of "
              "(o, m, l) partials per token and layer)", file=sys.stderr)
        return 2

    import libllmcpu_amd as nh
    from libllmcpu_amd import hip_rt

    if hip_rt.device_count() < 1:
        print("no HIP device", file=sys.stderr)
        return 1
    n_cu = hip_rt.attribute(ATTR_CU)
    clock_mhz = hip_rt.attribute(ATTR_CLOCK) / 1000.0

    log(f"[bench] allocating {N_LAYER} x {CTX}-row K/V buffers")
    kv = nh.KVCache([CTX] * N_LAYER, [KV_DIM] * N_LAYER, bf16=True)
    stream = kv.stream
    lib = nh.load_library()
    import ctypes as C

    # The cache's own buffers are filled through the device generator:
    # positions 0..CTX-1 of K (RMS-normed per head) and V, as appended. The
    # fill buffers (like everything else) are freed only after the last
    # timing: the driver clears freed device memory in the background, which
    # takes HBM bandwidth for seconds (decode measured 30.2 instead of 28.55
    # us per layer right after 8 GiB were freed).
    k_dev = hip_rt.malloc(CTX * KV_DIM * 4)
    v_dev = hip_rt.malloc(CTX * KV_DIM * 4)
    for li in range(N_LAYER):
        nh.fill_normal(k_dev, CTX * KV_DIM, (1234 + 3000 + li) * 256 + 1, HD, False, stream)
        nh.fill_normal(v_dev, CTX * KV_DIM, (1234 + 3000 + li) * 256 + 2, 0, False, stream)
        st = lib.nnc_hip_kv_append_f32_device(kv.handle, li, 0, CTX, C.c_void_p(k_dev), C.c_void_p(v_dev))
        if st:
            raise nh.NncError(st, lib.nnc_hip_last_error().decode())
        kv.sync()
    q_dec = hip_rt.malloc(N_LAYER * N_HEAD * HD * 4)
    o_dec = hip_rt.malloc(N_LAYER * N_HEAD * HD * 4)
    q_pre = hip_rt.malloc(N_LAYER * PROMPT * N_HEAD * HD * 4)
    o_pre = hip_rt.malloc(PROMPT * N_HEAD * HD * 4)
    for li in range(N_LAYER):
        nh.fill_normal(q_dec + li * N_HEAD * HD * 4, N_HEAD * HD, (1234 + 3000 + li) * 256, HD, False, stream)
        nh.fill_normal(q_pre + li * PROMPT * N_HEAD * HD * 4, PROMPT * N_HEAD * HD, (1234 + 3000 + li) * 256 + 3, HD,
                       False, stream)
    kv.sync()
    if args.calibrate:
        # A plain copy kernel of known size (torch's elementwise copy).
        import torch

        a = torch.ones(CALIBRATE_MIB << 18, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    def decode_step():
        for li in range(N_LAYER):
            kv.attend_device(li, q_dec + li * N_HEAD * HD * 4, o_dec + li * N_HEAD * HD * 4, n_tok=1, pos0=CTX - 1,
                             n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)

    def prefill_step():
        for li in range(N_LAYER):
            qb = q_pre + li * PROMPT * N_HEAD * HD * 4
            for c in range(PROMPT // CHUNK):
                kv.attend_device(li, qb + c * CHUNK * N_HEAD * HD * 4, o_pre + c * CHUNK * N_HEAD * HD * 4,
                                 n_tok=CHUNK, pos0=c * CHUNK, n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)

    def batch_step():
        # One forward pass of an nnc session (SESSION_BATCH tokens) at the end
        # of the context, through every layer.
        for li in range(N_LAYER):
            kv.attend_device(li, q_pre + li * PROMPT * N_HEAD * HD * 4, o_pre, n_tok=SESSION_BATCH,
                             pos0=CTX - SESSION_BATCH, n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)

    def timed(step, n):
        e0, e1 = hip_rt.Event(), hip_rt.Event()
        hip_rt.sync()
        w0 = time.perf_counter()
        e0.record(stream)
        for _ in range(n):
            step()
        e1.record(stream)
        e1.synchronize()
        hip_rt.sync()
        return e1.ms_since(e0), (time.perf_counter() - w0) * 1e3

    if args.only == "gemv":
        log(f"[bench] gemv {json.dumps(gemv_bench(nh, hip_rt, kv, stream, timed))}")
        return 0
    if args.only == "configs":
        from libllmcpu_amd import synth

        log(f"[bench] configs {json.dumps(configs_bench(nh, hip_rt, synth))}")
        return 0
    def prep_bench():
        # The pre-attention step (per-head RMSNorm of Q/K, RoPE, K/V append) at
        # the same shape, after the attention timings (it rewrites q and the
        # cache rows it appends): one token per layer, then 512-token chunks.
        k_in = hip_rt.malloc(CHUNK * KV_DIM * 4)
        v_in = hip_rt.malloc(CHUNK * KV_DIM * 4)
        gam = hip_rt.malloc(2 * HD * 4)
        nh.fill_normal(k_in, CHUNK * KV_DIM, 77, 0, False, stream)
        nh.fill_normal(v_in, CHUNK * KV_DIM, 78, 0, False, stream)
        hip_rt.to_device(gam, np.ones(2 * HD, np.float32))
        prep = nh.NncHipPrep(N_HEAD, N_KV, HD, gam, gam + HD * 4, 0, 1e-6, HD, 1000000.0, 1.0, 0, None)

        def prep_step(n_tok, pos0):
            for li in range(N_LAYER):
                kv.prep_append_device(li, q_pre + li * PROMPT * N_HEAD * HD * 4, k_in, v_in, pos0=pos0, n_tok=n_tok,
                                      prep=prep)

        prep_res = {}
        for label, n_tok, pos0 in (("decode", 1, CTX - 1), ("chunk", CHUNK, PROMPT - CHUNK)):
            prep_step(n_tok, pos0)
            ms, _ = timed(lambda: prep_step(n_tok, pos0), 10)
            us = ms * 1e3 / (10 * N_LAYER)
            prep_res[label] = {"n_tok": n_tok, "us_per_layer": round(us, 3), "bytes_per_layer": prep_bytes(n_tok),
                               "gbs": round(prep_bytes(n_tok) / (us * 1e-6) / 1e9, 1)}
        log(f"[bench] prep decode {prep_res['decode']['us_per_layer']} us/layer, "
            f"chunk {prep_res['chunk']['us_per_layer']} us/layer ({prep_res['chunk']['gbs']} GB/s)")
        for p_ in (k_in, v_in, gam):
            hip_rt.free(p_)
        return prep_res

    if args.only == "prep":
        prep_bench()
        return 0
    if args.only == "batch":
        batch_step()
        hip_rt.sync()
        b_ms, _ = timed(batch_step, 10)
        log(f"[bench] session batch {b_ms / 10:.4f} ms/step")
        return 0
    if args.only == "prefill":
        prefill_step()
        hip_rt.sync()
        pre_ms, _ = timed(prefill_step, args.prefill_steps)
        log(f"[bench] prefill {pre_ms / args.prefill_steps:.3f} ms/step")
        return 0
    log(f"[bench] decode warmup {args.warmup}")
    for _ in range(args.warmup):
        decode_step()
    hip_rt.sync()
    log(f"[bench] decode timed {args.steps} steps")
    dec_ms, dec_wall = timed(decode_step, args.steps)
    if args.only == "decode":
        log(f"[bench] decode {dec_ms / args.steps:.4f} ms/step")
        return 0
    dec_step_ms = dec_ms / args.steps
    dec_bytes = N_LAYER * decode_bytes(CTX)
    dec_gbs = dec_bytes / (dec_step_ms * 1e-3) / 1e9
    dec_launch_us = dec_ms * 1e3 / (args.steps * N_LAYER)
    dec_launch_gbs = decode_bytes(CTX) / (dec_launch_us * 1e-6) / 1e9

    log("[bench] prefill warmup 1")
    prefill_step()
    hip_rt.sync()
    log(f"[bench] prefill timed {args.prefill_steps} steps")
    pre_ms, pre_wall = timed(prefill_step, args.prefill_steps)
    pre_step_ms = pre_ms / args.prefill_steps
    pre_flops = N_LAYER * sum(prefill_flops(c * CHUNK, CHUNK) for c in range(PROMPT // CHUNK))
    pre_tflops = pre_flops / (pre_step_ms * 1e-3) / 1e12
    pre_launches = N_LAYER * (PROMPT // CHUNK)
    pre_launch_us = pre_ms * 1e3 / (args.prefill_steps * pre_launches)
    pre_launch_tflops = (pre_flops / pre_launches) / (pre_launch_us * 1e-6) / 1e12

    # nnc's "same bits whatever batch" (exact mode: every token on the split-K
    # kernel, bit-identical to its one-token call) for chunk 7 of every layer,
    # beside the prefill kernel on the same chunk.
    c7 = PROMPT // CHUNK - 1

    def chunk_step():
        for li in range(N_LAYER):
            qb = q_pre + li * PROMPT * N_HEAD * HD * 4
            kv.attend_device(li, qb + c7 * CHUNK * N_HEAD * HD * 4, o_pre + c7 * CHUNK * N_HEAD * HD * 4,
                             n_tok=CHUNK, pos0=c7 * CHUNK, n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)

    log("[bench] chunk 7: prefill kernel, then exact mode")
    chunk_step()
    hip_rt.sync()
    fast_ms, _ = timed(chunk_step, 3)
    lib.nnc_hip_kv_set_exact_batches(kv.handle, True)
    chunk_step()
    hip_rt.sync()
    exact_ms, _ = timed(chunk_step, 3)
    lib.nnc_hip_kv_set_exact_batches(kv.handle, False)
    exact_res = {"what": f"chunk {c7} of the {PROMPT}-token prompt ({CHUNK} tokens at keys 0 .. {PROMPT - 1}) "
                         "through every layer: the prefill kernel, and exact mode (nnc_hip_kv_set_exact_batches: "
                         "every token on the split-K kernel with its one-token bits)",
                 "prefill_kernel_us_per_layer": round(fast_ms * 1e3 / (3 * N_LAYER), 2),
                 "exact_us_per_layer": round(exact_ms * 1e3 / (3 * N_LAYER), 2),
                 "exact_over_prefill": round(exact_ms / fast_ms, 2),
                 "exact_tflops": round(prefill_flops(c7 * CHUNK, CHUNK) * 3 * N_LAYER / (exact_ms * 1e-3) / 1e12, 1)}
    log(f"[bench] exact mode {json.dumps(exact_res)}")

    # Parity samples, taken before the pre-attention benchmark rewrites q and
    # cache rows: layer 0's q and output of the timed decode step, and chunk 7
    # of layer 0 through the prefill kernel.
    width = N_HEAD * HD
    kv.attend_device(0, q_pre + c7 * CHUNK * width * 4, o_pre + c7 * CHUNK * width * 4, n_tok=CHUNK,
                     pos0=c7 * CHUNK, n_head=N_HEAD, n_kv=N_KV, head_dim=HD, scale=SCALE)
    kv.sync()
    samples = {"decode_q": hip_rt.to_host(np.empty((1, width), np.float32), q_dec),
               "decode_out": hip_rt.to_host(np.empty((1, width), np.float32), o_dec),
               "prefill_q": hip_rt.to_host(np.empty((CHUNK, width), np.float32), q_pre + c7 * CHUNK * width * 4),
               "prefill_out": hip_rt.to_host(np.empty((CHUNK, width), np.float32), o_pre + c7 * CHUNK * width * 4)}
    cache_l0 = kv.read(0, 0, CTX)

    log("[bench] session batch")
    batch_step()
    hip_rt.sync()
    b_ms, _ = timed(batch_step, 10)
    b_us = b_ms * 1e3 / (10 * N_LAYER)
    b_bytes = decode_bytes(CTX) + 2 * (SESSION_BATCH - 1) * N_HEAD * HD * 4
    log(f"[bench] session batch {b_us:.2f} us/layer")

    prep_res = prep_bench()

    log("[bench] gemv")
    gemv_res = gemv_bench(nh, hip_rt, kv, stream, timed)
    log(f"[bench] gemv {json.dumps(gemv_res)}")

    def traffic_of(path):
        tp = Path(path)
        if tp.exists():
            try:
                return json.loads(tp.read_text()).get("hbm_bytes_per_launch")
            except (ValueError, AttributeError):
                return None
        return None

    traffic = traffic_of(args.traffic)
    pre_traffic = traffic_of(args.prefill_traffic)

    log("[bench] host-buffer decode path")
    host_res = host_path_bench(nh, kv, q_dec, o_dec)
    log(f"[bench] host path {host_res['us_per_call']} us/call")

    cpu = None
    if not args.no_cpu:
        log(f"[bench] cpu baseline ~{args.cpu_seconds:.0f} s per setting")
        cpu = cpu_baseline(cache_l0, args.cpu_seconds, samples)

    configs = None
    if not args.no_configs:
        from libllmcpu_amd import synth

        log("[bench] other configurations")
        configs = configs_bench(nh, hip_rt, synth)
    kv.close()
    for p_ in (k_dev, v_dev, q_dec, o_dec, q_pre, o_pre):
        hip_rt.free(p_)

    line = {
        "metric": METRIC,
        "value": round(dec_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec_step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "qwen3-4b attention decode, 32768 cached keys, 36 layers (one token per step)",
                   "n_head": N_HEAD, "n_kv": N_KV, "head_dim": HD, "layers": N_LAYER, "context": CTX,
                   "kv_dtype": "bf16", "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "hbm", "achieved": round(dec_launch_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec_launch_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "decode_bf16_kernel<128,4,4,64,1,2> + decode_merge_kernel<128,4> (one attend call)",
                     "avg_launch_us": round(dec_launch_us, 3), "bytes_per_launch": decode_bytes(CTX)},
        "prefill": {"metric": "prefill-attn TFLOP/s", "value": round(pre_tflops, 1), "unit": "TFLOP/s",
                    "ms_per_step": round(pre_step_ms, 3), "steps": args.prefill_steps,
                    "workload": f"qwen3-4b prefill of {PROMPT} tokens in {CHUNK}-token chunks, 36 layers",
                    "roofline": {"bound": "mfma", "achieved": round(pre_launch_tflops, 1),
                                 "peak": MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                 "frac": round(pre_launch_tflops / MFMA_PEAK_TFLOPS, 4), "traffic": pre_traffic,
                                 "kernel": "prefill_kernel<128,4,2> (64 rows per work-group; Q as bf16 hi+lo against the "
                                           "bf16 K, fp16 P against the fp16 copy of V, fp32 accumulate)",
                                 "avg_launch_us": round(pre_launch_us, 3)}},
        "session_batch": {"what": f"one {SESSION_BATCH}-token forward pass of an nnc session (its batch size, "
                                  f"MTP verification included) ending at position {CTX - 1}, 36 layers; each token "
                                  "bit-identical to its one-token call (decode_bf16_multi_kernel)",
                          "ms_per_step": round(b_ms / 10, 4), "us_per_layer": round(b_us, 3),
                          "kv_gbs": round(b_bytes / (b_us * 1e-6) / 1e9, 1)},
        "prep": {"what": "per-head RMSNorm of Q and K, NEOX RoPE (base 1e6), BF16 K/V append, device memory",
                 "decode": prep_res["decode"], "chunk": prep_res["chunk"],
                 "roofline": {"bound": "hbm", "achieved": prep_res["chunk"]["gbs"], "peak": HBM_PEAK_GBS,
                              "unit": "GB/s", "frac": round(prep_res["chunk"]["gbs"] / HBM_PEAK_GBS, 4),
                              "kernel": "prep_kernel (512-token chunk)"}},
        "gemv": gemv_res,
        "host_path": host_res,
        "exact_mode": exact_res,
        "parity": cpu["parity"] if cpu else None,
        "configs": configs,
        "cpu_baseline": cpu,
        "device": {"cu": n_cu, "clock_mhz": clock_mhz},
        "wall_ms": {"decode": round(dec_wall, 2), "prefill": round(pre_wall, 2)},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

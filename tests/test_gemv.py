"""The weight gemvs on either side of attention (reference
src/libnnc/nn_ops.h:95-180, nn_ops.cpp:1000-1053, 1200-1316, 1352-1700):
BF16, Q8_0 split and Q4_S split weights, one activation vector or a batch of
up to 16.

CPU: the oracle's quantizers and block sums bit-exact against the reference
(vectors and compiled code), its gemvs against the reference's JIT kernels
and a float64 product of the dequantised weights, and closed forms. GPU: the
HIP gemvs against the oracle. Bound for every gemv comparison, per output:
|y - y_ref| <= 1e-5 * sum_k |w_rk x_k| (fp32 accumulation of the products;
the GPU's activations enter as bf16 hi + lo, 16 significant bits)."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"
REL = 1e-5


@pytest.fixture(scope="module")
def gold():
    return np.load(GOLDEN, allow_pickle=False)


def bf16_f32(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequant(fmt, w):
    """Float64 weights [rows, cols] from a layout tuple."""
    if fmt == "bf16":
        return bf16_f32(w[0]).astype(np.float64)
    if fmt == "q8_0":
        qs, sc = w
        return qs.astype(np.float64) * np.repeat(bf16_f32(sc).astype(np.float64), 32, axis=1)
    qs, sc, bi = w
    rows, half = qs.shape
    q = np.empty((rows, half * 2), np.float64)
    blocks = qs.reshape(rows, -1, 16)
    q.reshape(rows, -1, 32)[:, :, :16] = blocks & 15
    q.reshape(rows, -1, 32)[:, :, 16:] = blocks >> 4
    return q * np.repeat(bf16_f32(sc), 32, axis=1) + np.repeat(bf16_f32(bi), 32, axis=1)


def bound(fmt, w, x):
    return REL * (np.abs(x.astype(np.float64)) @ np.abs(dequant(fmt, w)).T) + 1e-30


def layouts(orc, wf):
    return {"bf16": (orc.bf16_round(wf),), "q8_0": orc.quantize_q8_0(wf), "q4_s": orc.quantize_q4_s(wf)}


def oracle_gemv(orc, fmt, w, x):
    return {"bf16": orc.gemv_bf16, "q8_0": orc.gemv_q8_0, "q4_s": orc.gemv_q4_s}[fmt](*w, x)


# ---- CPU: the oracle -------------------------------------------------------------------

def test_quantizers_and_block_sums_match_reference_vectors(orc, gold):
    w, x = gold["gemv/w"], gold["gemv/x"]
    for got, want in zip(orc.quantize_q8_0(w), (gold["gemv/q8_0/qs"], gold["gemv/q8_0/scales"])):
        assert np.array_equal(got, want)
    for got, want in zip(orc.quantize_q4_s(w),
                         (gold["gemv/q4_s/qs"], gold["gemv/q4_s/scales"], gold["gemv/q4_s/biases"])):
        assert np.array_equal(got, want)
    assert np.array_equal(orc.block_sums(x), gold["gemv/xsum"])


def test_gemvs_match_reference_vectors(orc, gold):
    w, x = gold["gemv/w"], gold["gemv/x"]
    lay = {"bf16": (orc.bf16_round(w),), "q8_0": (gold["gemv/q8_0/qs"], gold["gemv/q8_0/scales"]),
           "q4_s": (gold["gemv/q4_s/qs"], gold["gemv/q4_s/scales"], gold["gemv/q4_s/biases"])}
    for fmt, wl in lay.items():
        got = oracle_gemv(orc, fmt, wl, x)
        assert np.all(np.abs(got - gold[f"gemv/{fmt}/y"]) <= bound(fmt, wl, x)), fmt


def test_quantizers_and_gemvs_match_reference_code(orc, ref):
    rng = np.random.default_rng(11)
    for rows, cols, n in ((64, 256, 1), (260, 512, 3), (1024, 2560, 16)):
        wf = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        x = rng.standard_normal((n, cols)).astype(np.float32)
        for a, b in zip(orc.quantize_q8_0(wf), ref.quantize_q8_0(wf)):
            assert np.array_equal(a, b)
        for a, b in zip(orc.quantize_q4_s(wf), ref.quantize_q4_s(wf)):
            assert np.array_equal(a, b)
        assert np.array_equal(orc.block_sums(x), ref.block_sums(x))
        for fmt, wl in layouts(orc, wf).items():
            got = oracle_gemv(orc, fmt, wl, x)
            want = oracle_gemv(ref, fmt, wl, x)
            assert np.all(np.abs(got - want) <= bound(fmt, wl, x)), (fmt, rows, cols, n)


def test_gemvs_match_float64_product(orc):
    rng = np.random.default_rng(12)
    wf = (rng.standard_normal((96, 512)) * 0.1).astype(np.float32)
    x = rng.standard_normal((4, 512)).astype(np.float32)
    for fmt, wl in layouts(orc, wf).items():
        exact = x.astype(np.float64) @ dequant(fmt, wl).T
        assert np.all(np.abs(oracle_gemv(orc, fmt, wl, x) - exact) <= bound(fmt, wl, x)), fmt


def test_gemv_closed_forms(orc):
    # One weight per row: y_r = w_r * x_{k(r)} exactly; Q8_0 of a block holding
    # a single value v: scale = |v| / 127 rounded to BF16, q = +-127.
    cols, rows = 64, 8
    wf = np.zeros((rows, cols), np.float32)
    for r in range(rows):
        wf[r, 5 * r] = 0.25 * (r + 1) * (-1) ** r
    x = np.arange(cols, dtype=np.float32)[None, :] / 8
    y = orc.gemv_bf16(orc.bf16_round(wf), x)[0]
    assert np.array_equal(y, np.array([wf[r, 5 * r] * x[0, 5 * r] for r in range(rows)], np.float32))
    qs, sc = orc.quantize_q8_0(wf)
    assert all(abs(int(qs[r, 5 * r])) == 127 for r in range(rows))
    yq = orc.gemv_q8_0(qs, sc, x)[0]
    assert np.allclose(yq, y, rtol=1e-2)
    # Q4_S of a constant block: scale 0, bias = the value: y = v * (block sum of x).
    wc = np.full((2, 32), 0.5, np.float32)
    q4 = orc.quantize_q4_s(wc)
    assert np.all(q4[1] == 0) and np.all(bf16_f32(q4[2]) == 0.5)
    xc = np.ones((1, 32), np.float32)
    assert np.array_equal(orc.gemv_q4_s(*q4, xc)[0], np.array([16.0, 16.0], np.float32))


# ---- GPU: the HIP gemvs ------------------------------------------------------------------

GPU_SHAPES = [
    (256, 512, 1),      # one K split
    (4096, 2560, 1),    # Qwen3-4B q projection, decode
    (1024, 2560, 5),    # k / v projection, an MTP verification batch
    (2560, 9728, 16),   # MLP down, a full session batch (many K splits)
    (72, 96, 3),        # rows not a multiple of 16, three blocks
    (9728, 2560, 16),   # MLP gate / up
]
# seeded shapes beside them: any row count, columns any multiple of 32, 1-16 vectors
_rng = np.random.default_rng(2560)
GPU_SHAPES += [(int(_rng.integers(1, 3000)), 32 * int(_rng.integers(1, 320)), int(_rng.integers(1, 17))) for _ in range(8)]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,n", GPU_SHAPES, ids=[f"{r}x{c}x{n}" for r, c, n in GPU_SHAPES])
def test_hip_gemv_matches_oracle(orc, rows, cols, n):
    import libllmcpu_amd as nh

    rng = np.random.default_rng(rows * 7 + cols + n)
    wf = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    x = (rng.standard_normal((n, cols)) * 2).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        for fmt, wl in layouts(orc, wf).items():
            print(f"case gemv {fmt} {rows} x {cols}, {n} vectors", flush=True)
            got = kv.gemv(fmt, wl, x, rows=rows, cols=cols)
            want = oracle_gemv(orc, fmt, wl, x)
            err = np.abs(got.astype(np.float64) - want)
            b = bound(fmt, wl, x)
            print(f"  max |err| / bound {float((err / b).max()):.3f}", flush=True)
            assert np.all(err <= b), fmt
            if fmt == "q4_s":  # the caller's block sums instead of the kernel's
                got2 = kv.gemv(fmt, wl, x, rows=rows, cols=cols, xsum=orc.block_sums(x))
                assert np.array_equal(got2, got)


@pytest.mark.gpu
def test_hip_gemv_strides_and_errors(orc):
    import libllmcpu_amd as nh
    from libllmcpu_amd import hip_rt

    rows, cols, n = 48, 128, 3
    rng = np.random.default_rng(5)
    wf = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    qs, sc = orc.quantize_q8_0(wf)
    xs, ys = cols + 32, rows + 8
    xp = np.zeros((n, xs), np.float32)
    xp[:, :cols] = x
    dev = [hip_rt.malloc(a.nbytes) for a in (qs, sc, xp)]
    y_dev = hip_rt.malloc(n * ys * 4)
    try:
        for d, a in zip(dev, (qs, sc, xp)):
            hip_rt.to_device(d, a)
        hip_rt.to_device(y_dev, np.full((n, ys), 7.0, np.float32))
        with nh.KVCache([16], [64]) as kv:
            print("case gemv strides", flush=True)
            kv.gemv_device("q8_0", (dev[0], dev[1]), dev[2], y_dev, rows=rows, cols=cols, n_batch=n, x_stride=xs,
                           y_stride=ys)
            kv.sync()
            y = hip_rt.to_host(np.empty((n, ys), np.float32), y_dev)
            want = orc.gemv_q8_0(qs, sc, x)
            assert np.all(np.abs(y[:, :rows] - want) <= bound("q8_0", (qs, sc), x))
            assert np.all(y[:, rows:] == 7.0)  # the gap between output rows is untouched
            print("case gemv errors", flush=True)
            with pytest.raises(nh.NncError) as e:
                kv.gemv_device("q8_0", (dev[0], dev[1]), dev[2], y_dev, rows=rows, cols=cols - 16, n_batch=n)
            assert e.value.status == nh.NncStatus.UNSUPPORTED_MODEL
            with pytest.raises(nh.NncError) as e:
                kv.gemv_device("q8_0", (dev[0], dev[1]), dev[2], y_dev, rows=rows, cols=cols, n_batch=n,
                               x_stride=cols - 1)
            assert e.value.status == nh.NncStatus.INVALID_ARGUMENT
            kv.gemv_device("q8_0", (dev[0], dev[1]), dev[2], y_dev, rows=rows, cols=cols, n_batch=0)  # no-op
    finally:
        for d in dev + [y_dev]:
            hip_rt.free(d)


# (rows of each matrix, cols, vectors): q/k/v-like and gate/up-like groups, a
# last matrix with a partial 16-row tile, a batch over 16 vectors (two
# launches), a K range past one LDS copy (K splits), and a group whose first
# matrix has 40 rows (not a multiple of 16: run one matrix at a time).
GROUPS = [
    ((256, 64, 64), 512, 1),
    ((256, 64, 64), 512, 5),
    ((96, 96), 2560, 16),
    ((64, 32, 40), 256, 20),
    ((48, 16), 9728, 3),
    ((40, 64), 256, 1),
    ((40, 64), 256, 4),
]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols,n", GROUPS, ids=[f"{'+'.join(map(str, r))}x{c}x{n}" for r, c, n in GROUPS])
def test_hip_gemv_group_equals_single_calls(orc, rows, cols, n):
    """nnc_hip_gemv_group writes into each matrix's Y exactly the bits its
    single-matrix call writes (the same kernels and sums per row, the matrices
    stacked along the rows), for every format; each within the bound of the
    oracle too."""
    import libllmcpu_amd as nh
    from libllmcpu_amd import hip_rt

    rng = np.random.default_rng(sum(rows) + cols + n)
    wfs = [(rng.standard_normal((r, cols)) * 0.05).astype(np.float32) for r in rows]
    x = (rng.standard_normal((n, cols)) * 2).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        for fmt in ("bf16", "q8_0", "q4_s"):
            print(f"case gemv group {fmt} {rows} x {cols}, {n} vectors", flush=True)
            wls = [layouts(orc, wf)[fmt] for wf in wfs]
            dev = []
            try:
                def up(a):
                    a = np.ascontiguousarray(a)
                    d = hip_rt.malloc(max(a.nbytes, 16))
                    dev.append(d)
                    hip_rt.to_device(d, a)
                    return d

                w_dev = [tuple(up(a) for a in wl) for wl in wls]
                x_dev = up(x)
                y_grp = [up(np.full((n, r), 7.0, np.float32)) for r in rows]
                y_one = [up(np.full((n, r), 7.0, np.float32)) for r in rows]
                kv.gemv_group_device(fmt, [(w, y, r) for w, y, r in zip(w_dev, y_grp, rows)], x_dev, cols=cols,
                                     n_batch=n)
                for w, y, r in zip(w_dev, y_one, rows):
                    kv.gemv_device(fmt, w, x_dev, y, rows=r, cols=cols, n_batch=n)
                kv.sync()
                for m, (r, wl) in enumerate(zip(rows, wls)):
                    got = hip_rt.to_host(np.empty((n, r), np.float32), y_grp[m])
                    one = hip_rt.to_host(np.empty((n, r), np.float32), y_one[m])
                    assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), (fmt, m)
                    err = np.abs(got.astype(np.float64) - oracle_gemv(orc, fmt, wl, x))
                    assert np.all(err <= bound(fmt, wl, x)), (fmt, m)
            finally:
                for d in dev:
                    hip_rt.free(d)


@pytest.mark.gpu
def test_hip_gemv_group_strides_and_block_sums(orc):
    """A group with y_stride past each matrix's rows (the gap untouched) and X
    rows x_stride apart, and for Q4_S the caller's block sums: each Y equals its
    single-matrix call's bits."""
    import libllmcpu_amd as nh
    from libllmcpu_amd import hip_rt

    rows, cols, n = (64, 32), 256, 3
    xs = cols + 64
    rng = np.random.default_rng(77)
    wfs = [(rng.standard_normal((r, cols)) * 0.05).astype(np.float32) for r in rows]
    x = (rng.standard_normal((n, cols)) * 2).astype(np.float32)
    xp = np.zeros((n, xs), np.float32)
    xp[:, :cols] = x
    sums = orc.block_sums(x).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        for fmt in ("bf16", "q8_0", "q4_s"):
            print(f"case gemv group strides {fmt}", flush=True)
            wls = [layouts(orc, wf)[fmt] for wf in wfs]
            dev = []
            try:
                def up(a):
                    a = np.ascontiguousarray(a)
                    d = hip_rt.malloc(max(a.nbytes, 16))
                    dev.append(d)
                    hip_rt.to_device(d, a)
                    return d

                w_dev = [tuple(up(a) for a in wl) for wl in wls]
                x_dev, s_dev = up(xp), up(sums)
                ys = [r + 8 for r in rows]
                y_grp = [up(np.full((n, y), 7.0, np.float32)) for y in ys]
                y_one = [up(np.full((n, y), 7.0, np.float32)) for y in ys]
                q4 = fmt == "q4_s"
                kv.gemv_group_device(fmt, [(w, y, r, st) for w, y, r, st in zip(w_dev, y_grp, rows, ys)], x_dev,
                                     cols=cols, n_batch=n, x_stride=xs, xsum_dev=s_dev if q4 else 0,
                                     xsum_stride=cols // 32)
                for w, y, r, st in zip(w_dev, y_one, rows, ys):
                    kv.gemv_device(fmt, w, x_dev, y, rows=r, cols=cols, n_batch=n, x_stride=xs, y_stride=st,
                                   xsum_dev=s_dev if q4 else 0, xsum_stride=cols // 32)
                kv.sync()
                for m, (r, st) in enumerate(zip(rows, ys)):
                    got = hip_rt.to_host(np.empty((n, st), np.float32), y_grp[m])
                    one = hip_rt.to_host(np.empty((n, st), np.float32), y_one[m])
                    assert np.array_equal(got.view(np.uint32), one.view(np.uint32)), (fmt, m)
                    assert np.all(got[:, r:] == 7.0)  # the gap between output rows is untouched
                    assert np.all(np.abs(got[:, :r] - oracle_gemv(orc, fmt, wls[m], x)) <= bound(fmt, wls[m], x))
            finally:
                for d in dev:
                    hip_rt.free(d)


@pytest.mark.gpu
def test_hip_gemv_group_errors():
    import libllmcpu_amd as nh

    with nh.KVCache([16], [64]) as kv:
        print("case gemv group errors", flush=True)
        for bad in (dict(fmt="bf16", mats=[]), dict(fmt="bf16", mats=[((16,), 16, 16)] * 4)):
            with pytest.raises(nh.NncError) as e:
                kv.gemv_group_device(bad["fmt"], bad["mats"], 16, cols=32, n_batch=1)
            assert e.value.status == nh.NncStatus.INVALID_ARGUMENT
        with pytest.raises(nh.NncError) as e:  # Q8_0 without scales
            kv.gemv_group_device("q8_0", [((16,), 16, 16)], 16, cols=32, n_batch=1)
        assert e.value.status == nh.NncStatus.INVALID_ARGUMENT


# ---- the lm_head argmax (reference nn_ops.cpp:1055-1197, model.cpp:2181-2190) ----------

def bf16_rows(rng, rows, cols):
    """BF16 bits of uniform(-1, 1) weights, drawn as bit patterns (fast at lm_head sizes)."""
    mag = rng.integers(0x3C00, 0x3F80, size=(rows, cols), dtype=np.uint16)  # [2^-7, 1)
    return mag | (rng.integers(0, 2, size=(rows, cols), dtype=np.uint16) << 15)


def argmax_ok(w, x, got, want):
    """The reference test's criterion (tests.cpp:603-619): the same row, or rows
    whose float64 values are within 1e-3 * max(1, |best|)."""
    if got == want:
        return True
    if got < 0 or want < 0:
        return False
    y_got, y_want = (float(bf16_f32(w[r]).astype(np.float64) @ x.astype(np.float64)) for r in (got, want))
    return abs(y_got - y_want) <= 1e-3 * max(1.0, abs(y_want))


def test_argmax_matches_reference_vectors(orc, gold):
    for name in ("fast", "fallback"):
        w, x = gold[f"argmax/{name}/w"], gold[f"argmax/{name}/x"]
        assert orc.gemv_bf16_argmax(w, x) == int(gold[f"argmax/{name}/index"]), name


def test_argmax_matches_reference_code(orc, ref):
    # The reference test's shapes (tests.cpp:572-574) and larger ones, to its
    # criterion (the oracle sums the fp32 products in column order, the
    # reference's JIT kernel in its own order).
    rng = np.random.default_rng(0xA12A)
    for rows, cols in ((4, 32), (16, 256), (2048, 256), (256, 1536), (7, 5), (300, 64), (1024, 2560)):
        w = orc.bf16_round(rng.uniform(-1, 1, (rows, cols)).astype(np.float32))
        x = rng.uniform(-1, 1, cols).astype(np.float32)
        got, want = orc.gemv_bf16_argmax(w, x), ref.gemv_bf16_argmax(w, x)
        assert argmax_ok(w, x, got, want), (rows, cols, got, want)


def test_argmax_closed_forms(orc):
    rng = np.random.default_rng(3)
    w = bf16_rows(rng, 64, 32)
    x = np.ones(32, np.float32)
    assert orc.gemv_bf16_argmax(np.zeros((0, 32), np.uint16), x) == -1
    assert orc.gemv_bf16_argmax(w[:, :0], x[:0]) == -1
    # One row of all ones against x = 1 wins with 32; two copies: the first.
    w[40] = 0x3F80
    assert orc.gemv_bf16_argmax(w, x) == 40
    w[12] = 0x3F80
    assert orc.gemv_bf16_argmax(w, x) == 12
    # NaN rows are never chosen; all NaN (or all -inf): row 0.
    w[12] = 0x7FC0
    assert orc.gemv_bf16_argmax(w, x) == 40
    assert orc.gemv_bf16_argmax(np.full((8, 32), 0x7FC0, np.uint16), x) == 0
    assert orc.gemv_bf16_argmax(np.full((8, 32), 0xFF80, np.uint16), x) == 0  # -inf weights, y = -inf


GPU_ARGMAX_SHAPES = [
    (4, 32), (16, 256), (2048, 256), (256, 1536),  # the reference test's fast-path shapes
    (1001, 2560),  # rows not a multiple of 4 (nor of a work-group's rows)
    (151936, 2560),  # Qwen3-4B's lm_head (tied embeddings), 778 MB
]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,cols", GPU_ARGMAX_SHAPES, ids=[f"{r}x{c}" for r, c in GPU_ARGMAX_SHAPES])
def test_hip_gemv_argmax_matches_oracle(orc, rows, cols):
    import libllmcpu_amd as nh

    rng = np.random.default_rng(rows + cols)
    w = bf16_rows(rng, rows, cols)
    x = rng.uniform(-1, 1, cols).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        print(f"case argmax {rows} x {cols}", flush=True)
        got = kv.gemv_argmax(w, x)
        want = orc.gemv_bf16_argmax(w, x)
        print(f"  got {got}, oracle {want}", flush=True)
        assert argmax_ok(w, x, got, want)
        # Plant a tie with the winner at an earlier and a later row: the earlier wins.
        top = got
        early, late = (top // 3, min(rows - 1, top + 1 + (rows - top) // 2)) if rows > 2 else (0, rows - 1)
        if early != top and late != top:
            w[early] = w[top]
            w[late] = w[top]
            print(f"case argmax {rows} x {cols}, ties at {early}, {top}, {late}", flush=True)
            assert kv.gemv_argmax(w, x) == early


@pytest.mark.gpu
def test_hip_gemv_argmax_special_values(orc):
    import libllmcpu_amd as nh

    rng = np.random.default_rng(8)
    rows, cols = 4096, 256
    w = bf16_rows(rng, rows, cols)
    x = np.abs(rng.uniform(0.1, 1, cols)).astype(np.float32)  # positive: -inf weights give y = -inf
    with nh.KVCache([16], [64]) as kv:
        print("case argmax special values", flush=True)
        w[100] = 0x3F80  # the winner: 1.0 everywhere
        w[50] = 0x7FC0  # a NaN row is never chosen
        assert kv.gemv_argmax(w, x) == 100
        assert kv.gemv_argmax(np.full((rows, cols), 0x7FC0, np.uint16), x) == 0  # all NaN
        assert kv.gemv_argmax(np.full((rows, cols), 0xFF80, np.uint16), x) == 0  # all -inf
        wn = np.full((rows, cols), 0xFF80, np.uint16)
        wn[3000] = 0xBF80  # one finite row (-sum x) among -inf rows
        assert kv.gemv_argmax(wn, x) == 3000
        assert kv.gemv_argmax(w[:0], x) == -1
        print("case argmax errors", flush=True)
        with pytest.raises(nh.NncError) as e:
            kv.gemv_argmax(w[:, :48], x[:48])
        assert e.value.status == nh.NncStatus.UNSUPPORTED_MODEL


def test_vector_argmax_closed_forms(orc):
    # The quantised lm_head's scan (reference model.cpp:2192-2195): the first
    # strictly larger row from row 0.
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    assert orc.argmax_f32(np.array([], np.float32)) == 0
    assert orc.argmax_f32(np.array([1, 3, 2, 3], np.float32)) == 1
    assert orc.argmax_f32(np.array([nan, 3, 5], np.float32)) == 0  # row 0 NaN: nothing is larger
    assert orc.argmax_f32(np.array([1, nan, 5, nan], np.float32)) == 2
    assert orc.argmax_f32(np.array([-inf, -inf, -inf], np.float32)) == 0
    assert orc.argmax_f32(np.array([-inf, nan, -2], np.float32)) == 2
    rng = np.random.default_rng(4)
    for n in (2, 17, 1000):
        y = rng.standard_normal(n).astype(np.float32)
        y[rng.integers(1, n, n // 5 + 1)] = nan
        assert orc.argmax_f32(y) == int(np.nanargmax(y))  # first occurrence of the largest non-NaN


def test_argmax_fallback_row0_nan_matches_reference(orc, ref):
    # The reference's 4-row / threaded paths skip a NaN row 0, its fallback
    # (rows not a multiple of 4) keeps it; the oracle restates both.
    rng = np.random.default_rng(6)
    for rows in (7, 8, 1001, 1024):
        w = bf16_rows(rng, rows, 256)
        w[0] = 0x7FC0
        x = rng.uniform(-1, 1, 256).astype(np.float32)
        want = ref.gemv_bf16_argmax(w, x)
        assert orc.gemv_bf16_argmax(w, x) == want, rows
        assert (want == 0) == (rows % 4 != 0), rows


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 5, 1000, 151936, 262144])
def test_hip_argmax_f32_matches_oracle(orc, n):
    import libllmcpu_amd as nh

    rng = np.random.default_rng(n)
    y = rng.standard_normal(n).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        print(f"case argmax over {n} logits", flush=True)
        assert kv.argmax(y) == orc.argmax_f32(y)
        if n > 4:
            top = int(np.argmax(y))
            y[[n // 3, (2 * n) // 3]] = y[top]  # ties
            y[rng.integers(1, n, 3)] = np.nan
            y[top] = np.nan if top != 0 else y[top]
            print(f"case argmax over {n} logits, ties and NaN", flush=True)
            assert kv.argmax(y) == orc.argmax_f32(y)
            y[0] = np.nan
            assert kv.argmax(y) == orc.argmax_f32(y) == 0
            assert kv.argmax(np.full(n, -np.inf, np.float32)) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("rows", [7, 1000, 1001])
def test_hip_gemv_argmax_row0_nan(orc, rows):
    import libllmcpu_amd as nh

    rng = np.random.default_rng(rows)
    w = bf16_rows(rng, rows, 256)
    w[0] = 0x7FC0
    x = rng.uniform(-1, 1, 256).astype(np.float32)
    with nh.KVCache([16], [64]) as kv:
        print(f"case argmax {rows} x 256, row 0 NaN", flush=True)
        got, want = kv.gemv_argmax(w, x), orc.gemv_bf16_argmax(w, x)
        assert got == want if rows % 4 != 0 else argmax_ok(w, x, got, want)

"""GPU parity: the HIP path through the C ABI against the pinned oracle.

Bars:
  * dequantization, repack and top-k: bit-exact;
  * GEMV (f32 activations): against the f64 oracle, relative L2 <= 1e-4 and,
    per token, max |delta| <= 1e-3 * ||y_ref[token]||_2;
  * GEMM (x and dequantized W rounded to fp16, the reference's DRIFT/GEMM2
    rounding points): the same two bounds against the fp16-rounded oracle.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TYPES = ["Q8_0", "Q8_0R", "Q4_K", "Q6_K", "Q2_K", "IQ2_XXS"]
REL_L2 = 1e-4
ROW_FRAC = 1e-3


def check_close(y, ref, what):
    y = np.asarray(y, np.float64).reshape(ref.shape)
    d = y - ref
    rel = np.linalg.norm(d) / max(np.linalg.norm(ref), 1e-30)
    row_norm = np.linalg.norm(ref, axis=1)
    worst = np.max(np.abs(d), axis=1) / np.maximum(row_norm, 1e-30)
    print(f"{what}: rel_l2={rel:.2e} max_row_frac={worst.max():.2e}", flush=True)
    assert rel <= REL_L2, f"{what}: relative L2 {rel:.3e} > {REL_L2}"
    assert np.all(worst <= ROW_FRAC), f"{what}: max|d| / ||row|| {worst.max():.3e} > {ROW_FRAC}"


def make_weights(eff, tname, rows, k, seed):
    """(type code for the op, bytes to upload, GGUF bytes, n_blocks)."""
    base = "Q8_0" if tname == "Q8_0R" else tname
    w = eff.quantize(base, eff.fill_normal(seed, 0.02, rows * k))
    e, _ = eff.geometry(base)
    n = rows * k // e
    if tname == "Q8_0R":
        return eff.Q8_0R, eff.repack(w, n), w, n
    return eff.TYPES[tname], w, w, n


def upload_w(ctx, eff, tname, data, n):
    b = ctx.upload(data)
    if tname == "Q8_0R":
        b.mark_r(n)
    return b


def oracle_type(orc, tname):
    return orc.Q8_0 if tname == "Q8_0R" else orc.NAMES[tname]


# ---- dequantization --------------------------------------------------------------

@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("nrows", [1, 7, 1000])
def test_dequant_bit_exact(ctx, eff, orc, tname, nrows):
    k = 256
    t, data, gguf, n = make_weights(eff, tname, nrows, k, 3 + nrows)
    wb = upload_w(ctx, eff, tname, data, n)
    out = ctx.alloc(nrows * k * 4)
    ctx.dequant(t, wb, out, n)
    got = out.read(np.uint32)
    want = orc.dequant(oracle_type(orc, tname), gguf, n).view(np.uint32)
    assert np.array_equal(got, want)
    wb.free(); out.free()


def test_dequant_q8_0r_partial_call_uses_tensor_scales(ctx, eff, orc):
    """A call over fewer blocks than the tensor still finds the scales at 32N
    (the output head is called with the tokenizer's vocabulary, repack.js:254-259)."""
    t, data, gguf, n = make_weights(eff, "Q8_0R", 40, 256, 9)
    wb = upload_w(ctx, eff, "Q8_0R", data, n)
    out = ctx.alloc(100 * 32 * 4)
    ctx.dequant(t, wb, out, 100)
    assert np.array_equal(out.read(np.uint32), orc.dequant(orc.Q8_0, gguf, 100).view(np.uint32))


# ---- GEMV ----------------------------------------------------------------------

@pytest.fixture(params=["mx", "f32"])
def gemv_kernel(request, ctx, eff):
    """Both GEMV kernels: the int8 matrix-core one (default) and the f32 vector one."""
    ctx.set_option(eff.OPT_GEMV_KERNEL, 0 if request.param == "mx" else 1)
    yield request.param
    ctx.set_option(eff.OPT_GEMV_KERNEL, 0)


@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 8])
def test_gemv_vs_f64_oracle(ctx, eff, orc, gemv_kernel, tname, tokens):
    rows, k = 77, 2048      # rows not a multiple of the rows per wave; k split over two waves
    t, data, gguf, n = make_weights(eff, tname, rows, k, 20 + tokens)
    x = eff.fill_normal(1000 + tokens, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qgemv(t, wb, xb, yb, rows, k, tokens)
    ref = orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    check_close(yb.read(np.float32), ref, f"gemv[{gemv_kernel}] {tname} T={tokens}")
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("k", [32, 96, 192, 256, 768, 8192, 16384])
def test_gemv_k_edge_cases(ctx, eff, orc, gemv_kernel, k):
    """k = 32, 96: not a whole number of 64-weight tasks (f32 kernel); 192, 768:
    a pass of tasks partly beyond k; 8192, 16384: the largest per-wave slices."""
    for tname in (["Q8_0", "Q8_0R"] if k % 256 else TYPES):
        rows = 5
        t, data, gguf, n = make_weights(eff, tname, rows, k, k)
        x = eff.fill_normal(k + 1, 1.0, k)
        wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(rows * 4)
        ctx.qgemv(t, wb, xb, yb, rows, k, 1)
        check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, 1),
                    f"gemv[{gemv_kernel}] {tname} k={k}")


@pytest.mark.parametrize("tname", TYPES)
def test_gemv_x_dynamic_range(ctx, eff, orc, gemv_kernel, tname):
    """x digits are exact to 22 bits of each 32-value group's maximum: groups of
    zeros, of tiny (1e-30) and huge (1e30) values, outliers next to small values,
    and subnormals keep the f64 bounds."""
    rows, k, tokens = 40, 2048, 3
    t, data, gguf, n = make_weights(eff, tname, rows, k, 77)
    rng = np.random.default_rng(5)
    x = rng.normal(0, 1, (tokens, k)).astype(np.float32)
    x[0, :32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e30
    x[1, ::37] *= 1e4                                   # outliers among ordinary values
    x[1, 96:128] = np.float32(1e-40)                    # subnormal group
    x[2, :] *= 1e-3
    x = x.reshape(-1)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qgemv(t, wb, xb, yb, rows, k, tokens)
    ref = orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    check_close(yb.read(np.float32), ref, f"gemv[{gemv_kernel}] {tname} x range")


@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "IQ2_XXS"])
def test_gemv_non_finite_x(ctx, eff, gemv_kernel, tname):
    """A NaN or an infinity in x makes every output of its token non-finite (as
    an f32 dot product does); the other tokens are unaffected."""
    rows, k, tokens = 20, 512, 3
    t, data, gguf, n = make_weights(eff, tname, rows, k, 78)
    x = eff.fill_normal(79, 1.0, tokens * k).reshape(tokens, k)
    x[0, 100] = np.nan
    x[1, 300] = np.inf
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x.reshape(-1)), ctx.alloc(tokens * rows * 4)
    ctx.qgemv(t, wb, xb, yb, rows, k, tokens)
    y = yb.read(np.float32).reshape(tokens, rows)
    assert np.all(~np.isfinite(y[0])) and np.all(~np.isfinite(y[1])) and np.all(np.isfinite(y[2]))


# ---- the row GEMV for Q6_K matrices with many rows (the output projection) -------------

@pytest.mark.parametrize("rows,k", [(32768, 512), (32805, 4608), (40001, 2048), (32769, 8192), (32800, 2304),
                                      (33000, 768), (140001, 2048), (32800, 1024), (40001, 1536)])
def test_gemv_rows_q6_k_vs_f64_oracle(ctx, eff, orc, rows, k):
    """One token of a Q6_K matrix of >= 32768 rows runs the row kernel (a lane
    per half row-block): row counts that are not a multiple of the workgroups'
    rows (128 on average, 224 and 32 in the two halves of the grid from 8
    blocks per row), an odd number of blocks per row (block starts at both
    2-byte alignments in every column), k up to 32 blocks, more workgroups
    (1096) than the GPU holds at once, and the 4-slice form (k of 4 to 7
    blocks: 1024 and 1536)."""
    t, data, gguf, n = make_weights(eff, "Q6_K", rows, k, rows + k)
    x = eff.fill_normal(rows + 1, 1.0, k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.qmatmul(t, wb, xb, yb, rows, k, 1)
    check_close(yb.read(np.float32)[None, :], orc.gemv_f64(orc.Q6_K, gguf, rows, k, x, 1), f"rows Q6_K {rows}x{k}")
    for b in (wb, xb, yb):
        b.free()


def test_gemv_rows_q6_k_x_range_non_finite_and_fused(ctx, eff, orc):
    """The row kernel on x of mixed magnitudes (zeros, 1e-30, 1e30, outliers,
    subnormals) keeps the f64 bounds; a NaN or an infinity in x makes every
    output non-finite; fused launches over such a matrix are not applicable
    (their one-matrix GEMV is the row kernel)."""
    rows, k = 32800, 2048
    t, data, gguf, n = make_weights(eff, "Q6_K", rows, k, 91)
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, k).astype(np.float32)
    x[:32] = 0.0
    x[32:64] *= 1e-30
    x[64:96] *= 1e30
    x[200::37] *= 1e4
    x[96:128] = np.float32(1e-40)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.qgemv(t, wb, xb, yb, rows, k, 1)
    check_close(yb.read(np.float32)[None, :], orc.gemv_f64(orc.Q6_K, gguf, rows, k, x, 1), "rows Q6_K x range")
    for v in (np.nan, np.inf):
        x2 = eff.fill_normal(92, 1.0, k)
        x2[777] = v
        xb2 = ctx.upload(x2)
        ctx.qgemv(t, wb, xb2, yb, rows, k, 1)
        assert np.all(~np.isfinite(yb.read(np.float32)))
        xb2.free()
    y2 = ctx.alloc(rows * 4)
    with pytest.raises(eff.NotApplicable):
        ctx.qgemv_multi(t, eff.GEMV_SWIGLU, [wb, wb], xb, [yb], [rows, rows], k, 1)
    with pytest.raises(eff.NotApplicable):
        ctx.qgemv_multi(t, eff.GEMV_SECTIONS, [wb, wb], xb, [yb, y2], [rows, rows], k, 1)
    for b in (wb, xb, yb, y2):
        b.free()


def test_q8_0r_gemv_bit_identical_to_q8_0(ctx, eff):
    """Repacked and GGUF layouts give the same bits (kernels.wgsl.js:831-839)."""
    rows, k = 300, 2048
    _, data_r, gguf, n = make_weights(eff, "Q8_0R", rows, k, 5)
    x = eff.fill_normal(6, 1.0, 2 * k)
    a, b = ctx.upload(gguf), upload_w(ctx, eff, "Q8_0R", data_r, n)
    xb, ya, yb = ctx.upload(x), ctx.alloc(2 * rows * 4), ctx.alloc(2 * rows * 4)
    ctx.qgemv(eff.Q8_0, a, xb, ya, rows, k, 2)
    ctx.qgemv(eff.Q8_0R, b, xb, yb, rows, k, 2)
    assert np.array_equal(ya.read(np.uint32), yb.read(np.uint32))


# ---- GEMM --------------------------------------------------------------------------

@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("tokens", [64, 100, 200, 300, 1100])
def test_gemm_vs_fp16_oracle(ctx, eff, orc, tname, tokens):
    """Every tile configuration: 128 x 32 (< 256 tokens), 128 x 128 with a
    k split (>= 256), 256 x 128 (>= 1024; Q6_K stays on 128 x 128); Q8_0 from
    256 tokens on 128 x 128 tiles (300) and 256 x 256 (1100); rows and tokens
    not multiples of the tiles."""
    rows, k = 130, 512
    t, data, gguf, n = make_weights(eff, tname, rows, k, 40 + tokens)
    x = eff.fill_normal(2000 + tokens, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    ref = orc.gemm_f16(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    check_close(yb.read(np.float32), ref, f"gemm {tname} M={tokens}")
    for b in (wb, xb, yb):
        b.free()


def test_gemm_q8_0_k_not_multiple_of_step(ctx, eff, orc):
    rows, k, tokens = 64, 96, 70
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 71)
    x = eff.fill_normal(72, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    check_close(yb.read(np.float32), orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens), "gemm Q8_0 k=96")


@pytest.mark.parametrize("tokens,k", [(300, 544), (777, 544), (300, 96)])
def test_gemm_q8_0_tile_configs_same_bits(ctx, eff, orc, tokens, k):
    """Every Q8_0 tile configuration (EFF_OPT_GEMM_CONFIG 1..6: 256 x 256,
    128 x 128 with 3 and 6 stages, 64 x 128, 128 x 256, 256 x 128 on 2 x 2
    waves) sums each output in the same k order: the same bits as the
    automatic choice, and the fp16-rounded oracle's values. Rows and tokens
    are not multiples of any tile, k ends in half a step (k % 64 = 32), and
    k = 96 has fewer steps than the deepest pipeline has stages."""
    rows = 600
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 810 + tokens)
    x = eff.fill_normal(811 + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    y0 = yb.read(np.uint32)
    check_close(y0.view(np.float32), orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens), f"gemm Q8_0 M={tokens}")
    try:
        for cfg in range(1, 7):
            ctx.set_option(eff.OPT_GEMM_CONFIG, cfg)
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
            y = yb.read(np.uint32)
            assert np.array_equal(y, y0), f"config {cfg}: {np.count_nonzero(y != y0)} outputs differ"
        with pytest.raises(eff.EffError):
            ctx.set_option(eff.OPT_GEMM_CONFIG, 7)
        # 256 x 256 tiles take no k slices: a forced count leaves the bits
        ctx.set_option(eff.OPT_GEMM_CONFIG, 1)
        ctx.set_option(eff.OPT_GEMM_SPLIT, 3)
        yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
        ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
        assert np.array_equal(yb.read(np.uint32), y0)
    finally:
        ctx.set_option(eff.OPT_GEMM_CONFIG, 0)
        ctx.set_option(eff.OPT_GEMM_SPLIT, 0)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tokens,k", [(300, 4096), (200, 4064), (1600, 2080)])
def test_gemm_q8_0_k_slices(ctx, eff, orc, tokens, k):
    """Few rows and a long k: the tiles leave CUs idle and k is cut into
    slices over workgroups (25 tiles of 64 x 128 at 300 tokens: 8 slices;
    4064 ends in half a step inside the last slice; at 1600 tokens 125 tiles
    of 64 x 128 take 33 steps in slices of 17 and 16). The last workgroup of
    a tile adds the slices in slice order:
    every tile configuration gives the automatic choice's bits, a second call
    the same bits (the arrival counters start from zero again), and forced
    slice counts (EFF_OPT_GEMM_SPLIT) stay within the fp16 oracle's bound."""
    rows = 600
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 860 + tokens)
    x = eff.fill_normal(861 + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ref = orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens)
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    y0 = yb.read(np.uint32)
    check_close(y0.view(np.float32), ref, f"gemm Q8_0 M={tokens} k={k}")
    try:
        for cfg in (0, 1, 2, 3, 4, 5, 6):
            ctx.set_option(eff.OPT_GEMM_CONFIG, cfg)
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
            y = yb.read(np.uint32)
            assert np.array_equal(y, y0), f"config {cfg}: {np.count_nonzero(y != y0)} outputs differ"
        ctx.set_option(eff.OPT_GEMM_CONFIG, 0)
        for ks in (1, 2, 3, 64):
            ctx.set_option(eff.OPT_GEMM_SPLIT, ks)
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
            check_close(yb.read(np.float32), ref, f"gemm Q8_0 M={tokens} k={k} slices={ks}")
        with pytest.raises(eff.EffError):
            ctx.set_option(eff.OPT_GEMM_SPLIT, 65)
    finally:
        ctx.set_option(eff.OPT_GEMM_CONFIG, 0)
        ctx.set_option(eff.OPT_GEMM_SPLIT, 0)
    for b in (wb, xb, yb):
        b.free()


def test_gemm_q8_0_k_slices_graph_replays(ctx, eff, orc):
    """A recorded k-sliced GEMM (the x conversion and the product) replayed
    several times, with eager products of another shape between the replays
    (which use the same counters): every replay gives the eager bits."""
    rows, k, tokens = 520, 4096, 260
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 870)
    x = eff.fill_normal(871, 1.0, tokens * k)
    wb, xb, yb, y2 = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4), ctx.alloc(tokens * rows * 4)
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    y0 = yb.read(np.uint32)
    check_close(y0.view(np.float32), orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens), "gemm k slices")
    ctx.graph_begin()
    ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
    g = ctx.graph_end()
    try:
        for r in range(4):
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            g.launch()
            ctx.sync()
            y = yb.read(np.uint32)
            assert np.array_equal(y, y0), f"replay {r}: {np.count_nonzero(y != y0)} outputs differ"
            ctx.qgemm(t, wb, xb, y2, rows // 2, k, 200)   # another tile count on the same counters
    finally:
        g.destroy()
    for b in (wb, xb, yb, y2):
        b.free()


def test_set_stream_orders_after_the_previous_stream(ctx, eff):
    """Calls after eff_set_stream wait for those queued on the previous
    stream, with which they share the context's scratch (here two k-sliced
    GEMMs of different tile counts on the same arrival counters): a product
    queued on the context's stream, a switch to a caller's stream without a
    sync, another product there, and the switch back; both outputs keep the
    bits they have on one stream."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so.7")   # the runtime the library already loaded
    side = ctypes.c_void_p()
    assert hip.hipStreamCreateWithFlags(ctypes.byref(side), ctypes.c_uint(1)) == 0   # non-blocking, default priority
    k = 4096
    shapes = [(600, 300), (520, 200)]   # rows, tokens: 25 and 20 tiles of 64 x 128, k in 8 slices
    bufs, want = [], []
    for i, (rows, tokens) in enumerate(shapes):
        t, data, _, _ = make_weights(eff, "Q8_0", rows, k, 875 + i)
        wb, xb = ctx.upload(data), ctx.upload(eff.fill_normal(876 + i, 1.0, tokens * k))
        yb = ctx.alloc(tokens * rows * 4)
        ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
        want.append(yb.read(np.uint32))
        bufs.append((t, wb, xb, yb, rows, tokens))
    for rnd in range(3):
        for (_, _, _, yb, rows, tokens) in bufs:
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
        t, wb, xb, yb, rows, tokens = bufs[0]
        ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
        ctx.set_stream(side.value)
        t, wb, xb, yb, rows, tokens = bufs[1]
        ctx.qgemm(t, wb, xb, yb, rows, k, tokens)
        ctx.set_stream(None)
        for (_, _, _, yb, _, _), w in zip(bufs, want):
            assert np.array_equal(yb.read(np.uint32), w), rnd
    ctx.sync()
    assert hip.hipStreamSynchronize(side) == 0 and hip.hipStreamDestroy(side) == 0
    for (_, wb, xb, yb, _, _) in bufs:
        for b in (wb, xb, yb):
            b.free()


@pytest.mark.parametrize("tokens", [64, 100, 128])
def test_gemm_q8_0_from_64_tokens_over_many_rows(ctx, eff, orc, tokens):
    """From 64 tokens the router runs the tiled Q8_0 GEMM at every row count
    (6200 rows: the general kernel's 32-row tiles would be 194 workgroups):
    the fp16 oracle's values, Q8_0R's bits equal to Q8_0's, and every forced
    tile configuration the automatic choice's bits; k ends in half a step."""
    rows, k = 6200, 2080
    _, data, gguf, n = make_weights(eff, "Q8_0R", rows, k, 880 + tokens)
    x = eff.fill_normal(881 + tokens, 1.0, tokens * k)
    wq, wr = ctx.upload(gguf), upload_w(ctx, eff, "Q8_0R", data, n)
    xb, y0, y1 = ctx.upload(x), ctx.alloc(tokens * rows * 4), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()
    ctx.qmatmul(eff.Q8_0, wq, xb, y0, rows, k, tokens)
    assert ctx.stats()["gemm"] == before["gemm"] + 1
    ref = y0.read(np.uint32)
    check_close(ref.view(np.float32), orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens), f"gemm Q8_0 M={tokens}")
    try:
        for cfg in range(0, 7):
            ctx.set_option(eff.OPT_GEMM_CONFIG, cfg)
            for t, w in ((eff.Q8_0, wq), (eff.Q8_0R, wr)):
                y1.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
                ctx.qmatmul(t, w, xb, y1, rows, k, tokens)
                got = y1.read(np.uint32)
                assert np.array_equal(got, ref), f"type {t} config {cfg}: {np.count_nonzero(got != ref)} differ"
    finally:
        ctx.set_option(eff.OPT_GEMM_CONFIG, 0)
    for b in (wq, wr, xb, y0, y1):
        b.free()


@pytest.mark.parametrize("tokens,k", [(256, 2048), (300, 544), (777, 1024), (1100, 96), (2048, 512)])
def test_gemm_q8_0r_same_bits_as_q8_0(ctx, eff, tokens, k):
    """The prefill GEMM over a repacked tensor (Q8_0R: quants and scales in
    two regions, staged into the same LDS rows) gives the bits of the Q8_0
    tensor it was repacked from, in every tile configuration; k ends in half
    a step (544: the second block of the last step is absent) or has fewer
    steps than the pipeline has stages (96)."""
    rows = 600
    _, data, gguf, n = make_weights(eff, "Q8_0R", rows, k, 830 + tokens + k)
    x = eff.fill_normal(831 + tokens, 1.0, tokens * k)
    wq = ctx.upload(gguf)
    wr = upload_w(ctx, eff, "Q8_0R", data, n)
    xb, y0, y1 = ctx.upload(x), ctx.alloc(tokens * rows * 4), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()["gemm"]
    ctx.qmatmul(eff.Q8_0, wq, xb, y0, rows, k, tokens)
    ref = y0.read(np.uint32)
    try:
        for cfg in range(0, 7):
            ctx.set_option(eff.OPT_GEMM_CONFIG, cfg)
            y1.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            ctx.qmatmul(eff.Q8_0R, wr, xb, y1, rows, k, tokens)
            got = y1.read(np.uint32)
            assert np.array_equal(got, ref), f"config {cfg}: {np.count_nonzero(got != ref)} outputs differ"
    finally:
        ctx.set_option(eff.OPT_GEMM_CONFIG, 0)
    assert ctx.stats()["gemm"] == before + 8
    for b in (wq, wr, xb, y0, y1):
        b.free()


# ---- fused decode GEMV (gemv.gateUp, gemv.secciones) -----------------------------------

def silu64(v):
    v = np.asarray(v, np.float64)
    return v / (1.0 + np.exp(-v))


@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("tokens", [1, 2, 3])
def test_fused_gate_up(ctx, eff, orc, tname, tokens):
    """silu(W_gate x) * (W_up x) in one launch: against the f64 oracle, and
    against silu applied to the two one-matrix GEMVs' outputs (the same sums)."""
    rows, k = 300, 2048
    tg, dg, gg, n = make_weights(eff, tname, rows, k, 60 + tokens)
    _, du, gu, _ = make_weights(eff, tname, rows, k, 61 + tokens)
    x = eff.fill_normal(62 + tokens, 1.0, tokens * k)
    wg, wu, xb = upload_w(ctx, eff, tname, dg, n), upload_w(ctx, eff, tname, du, n), ctx.upload(x)
    y, yg, yu = (ctx.alloc(tokens * rows * 4) for _ in range(3))
    before = ctx.stats()["fused"]
    t = tg
    ctx.qgemv_multi(t, eff.GEMV_SWIGLU, [wg, wu], xb, [y], [rows, rows], k, tokens)
    assert ctx.stats()["fused"] == before + 1
    ctx.qgemv(t, wg, xb, yg, rows, k, tokens)
    ctx.qgemv(t, wu, xb, yu, rows, k, tokens)
    got = y.read(np.float32)
    g32, u32 = yg.read(np.float32), yu.read(np.float32)
    want = (g32 / (np.float32(1) + np.exp(-g32))) * u32
    assert np.allclose(got, want, rtol=4e-6, atol=0), f"max rel {np.max(np.abs(got - want) / np.abs(want)):.2e}"
    ot = oracle_type(orc, tname)
    ref = silu64(orc.gemv_f64(ot, gg, rows, k, x, tokens)) * orc.gemv_f64(ot, gu, rows, k, x, tokens)
    check_close(got, ref, f"gate+up {tname} T={tokens}")
    for b in (wg, wu, xb, y, yg, yu):
        b.free()


@pytest.mark.parametrize("tname", TYPES)
@pytest.mark.parametrize("n", [2, 3, 4])
def test_fused_sections_same_bits(ctx, eff, orc, tname, n):
    """2-4 matrices of one shape sharing x: each output is bit-identical to the
    one-matrix GEMV of that matrix."""
    rows, k, tokens = 130, 1024, 2
    ws, ggufs = [], []
    for i in range(n):
        t, d, g, nb = make_weights(eff, tname, rows, k, 70 + i)
        ws.append(upload_w(ctx, eff, tname, d, nb))
        ggufs.append(g)
    x = eff.fill_normal(75, 1.0, tokens * k)
    xb = ctx.upload(x)
    ys = [ctx.alloc(tokens * rows * 4) for _ in range(n)]
    ctx.qgemv_multi(t, eff.GEMV_SECTIONS, ws, xb, ys, [rows] * n, k, tokens)
    for i in range(n):
        y1 = ctx.alloc(tokens * rows * 4)
        ctx.qgemv(t, ws[i], xb, y1, rows, k, tokens)
        assert np.array_equal(ys[i].read(np.uint32), y1.read(np.uint32)), f"section {i}"
        check_close(ys[i].read(np.float32), orc.gemv_f64(oracle_type(orc, tname), ggufs[i], rows, k, x, tokens),
                    f"sections {tname} {i}/{n}")
        y1.free()


@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "Q6_K", "IQ2_XXS"])
def test_fused_sections_mixed_rows(ctx, eff, orc, tname):
    """Q, K, V and gate-like sections of different rows (2048 + 512 + 512 + 77):
    every output meets the f64 bar, and the launch count is one."""
    k, tokens, rows = 2048, 1, [2048, 512, 512, 77]
    ws, ggufs = [], []
    for i, r in enumerate(rows):
        t, d, g, nb = make_weights(eff, tname, r, k, 80 + i)
        ws.append(upload_w(ctx, eff, tname, d, nb))
        ggufs.append(g)
    x = eff.fill_normal(85, 1.0, tokens * k)
    xb = ctx.upload(x)
    ys = [ctx.alloc(tokens * r * 4) for r in rows]
    before = ctx.stats()
    ctx.qgemv_multi(t, eff.GEMV_SECTIONS, ws, xb, ys, rows, k, tokens)
    after = ctx.stats()
    assert after["fused"] == before["fused"] + 1 and after["gemv"] == before["gemv"]
    for i, r in enumerate(rows):
        check_close(ys[i].read(np.float32), orc.gemv_f64(oracle_type(orc, tname), ggufs[i], r, k, x, tokens),
                    f"sections {tname} rows={r}")


def test_fused_not_applicable_and_errors(ctx, eff):
    rows, k = 64, 512
    t, d, g, nb = make_weights(eff, "Q4_K", rows, k, 90)
    w, w2 = ctx.upload(d), ctx.upload(d)
    xb, y = ctx.alloc(4 * k * 4), ctx.alloc(4 * rows * 4)
    with pytest.raises(eff.NotApplicable):      # one matrix
        ctx.qgemv_multi(t, eff.GEMV_SECTIONS, [w], xb, [y], [rows], k, 1)
    with pytest.raises(eff.NotApplicable):      # four tokens
        ctx.qgemv_multi(t, eff.GEMV_SECTIONS, [w, w2], xb, [y, y], [rows, rows], k, 4)
    with pytest.raises(eff.NotApplicable):      # gate + up takes two matrices
        ctx.qgemv_multi(t, eff.GEMV_SWIGLU, [w, w2, w], xb, [y], [rows, rows, rows], k, 1)
    ctx.set_option(eff.OPT_GEMV_KERNEL, 1)
    try:
        with pytest.raises(eff.NotApplicable):  # the f32 vector GEMV has no fused form
            ctx.qgemv_multi(t, eff.GEMV_SWIGLU, [w, w2], xb, [y], [rows, rows], k, 1)
    finally:
        ctx.set_option(eff.OPT_GEMV_KERNEL, 0)
    with pytest.raises(eff.EffError) as e:
        ctx.qgemv_multi(t, eff.GEMV_SWIGLU, [w, w2], xb, [y], [rows, rows // 2], k, 1)
    assert e.value.code == eff.E_SHAPE
    with pytest.raises(eff.EffError) as e:
        ctx.qgemv_multi(t, eff.GEMV_SECTIONS, [w, w2], xb, [y, y], [rows, rows], 300, 1)
    assert e.value.code == eff.E_SHAPE


# ---- split-x product (Q2_K, Q4_K, IQ2_XXS, Q8_0, Q6_K; by default from 5 tokens for Q2_K and IQ2_XXS,
# from 9 for the others, from 4 here) ----

@pytest.fixture
def split_from_4(ctx, eff):
    """The split-x product at every token count it accepts (4 and up)."""
    ctx.set_option(eff.OPT_SPLIT_MIN_TOKENS, 4)
    yield
    ctx.set_option(eff.OPT_SPLIT_MIN_TOKENS, 0)


SPLIT_TYPES = ["Q2_K", "Q4_K", "IQ2_XXS"]


@pytest.mark.parametrize("tname,tokens", [("Q8_0", t) for t in (4, 7, 9, 16, 17, 32, 33, 63)] +
                         [("Q6_K", t) for t in (4, 7, 9, 16, 17, 33, 64, 100, 129)])
@pytest.mark.parametrize("k", [2048, 2304])
def test_split_x_per_block_scales_vs_f64_oracle(ctx, eff, orc, tname, tokens, k, split_from_4):
    """The split-x product of the types folded per group of steps (Q8_0: a
    scale per 32 weights, Q6_K: per 16) is f32-accurate at 1 and 2 token tiles
    and several token groups; rows not a multiple of 32; k = 2304 gives Q6_K
    rows starting 2 bytes past a dword (an odd number of 210-byte blocks)."""
    rows = 77
    t, data, gguf, n = make_weights(eff, tname, rows, k, 700 + tokens + k)
    x = eff.fill_normal(7000 + tokens + k, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()["split"]
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    assert ctx.stats()["split"] == before + 1
    check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"split-x {tname} M={tokens} k={k}")
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tokens,k", [(9, 2048), (17, 2304), (33, 2048), (63, 4096)])
def test_split_x_q8_0r_same_bits_as_q8_0(ctx, eff, tokens, k):
    """The split-x product over a repacked tensor (Q8_0R: each staged row is
    its 256 quant bytes from the quant region and 8 scales from the scale
    region) gives the bits of the Q8_0 tensor it was repacked from, through
    the router (9 to 63 tokens) and from an x prepared for the Q8_0 product
    (one layout for both)."""
    rows = 130
    _, data, gguf, n = make_weights(eff, "Q8_0R", rows, k, 860 + tokens + k)
    x = eff.fill_normal(861 + tokens, 1.0, tokens * k)
    wq, wr = ctx.upload(gguf), upload_w(ctx, eff, "Q8_0R", data, n)
    xb, y0, y1 = ctx.upload(x), ctx.alloc(tokens * rows * 4), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()["split"]
    ctx.qmatmul(eff.Q8_0, wq, xb, y0, rows, k, tokens)
    ctx.qmatmul(eff.Q8_0R, wr, xb, y1, rows, k, tokens)
    assert ctx.stats()["split"] == before + 2
    ref = y0.read(np.uint32)
    assert np.array_equal(y1.read(np.uint32), ref)
    nb, lay = ctx.qmatmul_x_layout(eff.Q8_0R, rows, k, tokens)
    assert lay == 0x100 and (nb, lay) == ctx.qmatmul_x_layout(eff.Q8_0, rows, k, tokens)
    xp = ctx.alloc(nb)
    ctx.qmatmul_prepare_x(eff.Q8_0, xb, xp, rows, k, tokens)
    y1.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
    ctx.qmatmul_prepared(eff.Q8_0R, wr, xp, y1, rows, k, tokens)
    assert np.array_equal(y1.read(np.uint32), ref)
    for b in (wq, wr, xb, y0, y1, xp):
        b.free()


@pytest.mark.parametrize("tname", SPLIT_TYPES)
@pytest.mark.parametrize("tokens", [4, 7, 16, 17, 33, 64, 100, 129])
def test_split_x_vs_f64_oracle(ctx, eff, orc, tname, tokens, split_from_4):
    """f32 accuracy at every token count: 1, 2 and 4 token tiles per wave and
    several token groups; rows not a multiple of the 32/64-row tiles; k = 2304
    (9 blocks: waves with one and with two blocks, odd IQ2_XXS block offsets)."""
    rows, k = 77, 2304
    t, data, gguf, n = make_weights(eff, tname, rows, k, 300 + tokens)
    x = eff.fill_normal(3000 + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()["split"]
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    assert ctx.stats()["split"] == before + 1
    check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"split-x {tname} M={tokens}")
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tname", SPLIT_TYPES)
@pytest.mark.parametrize("k", [256, 512, 8192])
def test_split_x_k_and_configs(ctx, eff, orc, tname, k):
    """One block per row, fewer blocks than waves, many blocks per wave; every
    workgroup configuration (32 rows x 8 waves, 64 rows x 4 waves, and the same
    with k in two slices over two workgroups) meets the bar."""
    rows, tokens = 100, 20
    t, data, gguf, n = make_weights(eff, tname, rows, k, 400 + k)
    x = eff.fill_normal(4000 + k, 1.0, tokens * k)
    wb, xb = ctx.upload(data), ctx.upload(x)
    ref = orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    for cfg in (1, 2, 3):
        yb = ctx.alloc(tokens * rows * 4)
        ctx.set_option(eff.OPT_SPLIT_CONFIG, cfg)
        try:
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
        finally:
            ctx.set_option(eff.OPT_SPLIT_CONFIG, 0)
        got = yb.read(np.uint32)
        check_close(got.view(np.float32), ref, f"split-x {tname} k={k} cfg={cfg}")
        if cfg == 3:    # two slices' sums added in slice order: the same bits on every call
            ctx.set_option(eff.OPT_SPLIT_CONFIG, cfg)
            try:
                ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
            finally:
                ctx.set_option(eff.OPT_SPLIT_CONFIG, 0)
            assert np.array_equal(yb.read(np.uint32), got)
        yb.free()


@pytest.mark.parametrize("tname", SPLIT_TYPES + ["Q8_0", "Q8_0R", "Q6_K"])
@pytest.mark.parametrize("tokens", [9, 40, 130])
def test_split_x_k_slices(ctx, eff, orc, tname, tokens):
    """k slices over workgroups (EFF_OPT_SPLIT_SLICES 2, 3, 7 and 64, more
    than the 33 blocks of k: one block per slice, some slices empty of
    blocks for a wave): each meets the f64 bar, and a second call gives the
    same bits (the tile's last workgroup adds the slices in slice order and
    leaves the arrival counters at zero)."""
    rows, k = 200, 8448
    t, data, gguf, n = make_weights(eff, tname, rows, k, 880 + tokens)
    x = eff.fill_normal(881 + tokens, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ref = orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    gemm_min = 64 if tname in ("Q8_0", "Q8_0R") and tokens >= 64 else None
    try:
        if gemm_min:
            ctx.set_option(eff.OPT_GEMM_MIN_TOKENS, 1000)   # Q8_0 beyond 63 tokens: split-x too
        for ks in (2, 3, 7, 64):
            ctx.set_option(eff.OPT_SPLIT_SLICES, ks)
            before = ctx.stats()["split"]
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
            assert ctx.stats()["split"] == before + 1
            y0 = yb.read(np.uint32)
            check_close(y0.view(np.float32), ref, f"split-x {tname} M={tokens} slices={ks}")
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
            assert np.array_equal(yb.read(np.uint32), y0), f"slices={ks}: a second call differs"
        with pytest.raises(eff.EffError):
            ctx.set_option(eff.OPT_SPLIT_SLICES, 65)
    finally:
        ctx.set_option(eff.OPT_SPLIT_SLICES, 0)
        if gemm_min:
            ctx.set_option(eff.OPT_GEMM_MIN_TOKENS, gemm_min)
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tname", SPLIT_TYPES + ["Q8_0", "Q6_K"])
@pytest.mark.parametrize("tokens,k,split", [(3, 16384, True), (2, 32768, True), (2, 14336, False),
                                            (6, 8192, True), (4, 8192, False)])
def test_router_split_x_where_gemv_digits_do_not_fit(ctx, eff, orc, tname, tokens, k, split):
    """Where the int8 matrix-core GEMVs cannot hold x's digits in LDS (3.5
    bytes per token and k: 3 tokens at k = 16384, 2 at 32768, 6 at 8192),
    the router takes the split-x product from 2 tokens instead of the f32
    vector GEMV; where they fit (2 tokens at 14336, 4 at 8192) the GEMV
    stays. Both meet the f64 bar."""
    rows = 300
    t, data, gguf, n = make_weights(eff, tname, rows, k, 890 + tokens + k)
    x = eff.fill_normal(891 + tokens, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    after = ctx.stats()
    assert after["split"] - before["split"] == (1 if split else 0)
    check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"router {tname} M={tokens} k={k}")
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tname", ["Q8_0", "Q4_K", "Q6_K"])
@pytest.mark.parametrize("tokens,k,rows,split", [(7, 4608, 300, True), (8, 5120, 300, True), (8, 4096, 300, False),
                                                 (6, 4608, 300, False), (7, 4096, 5200, None)])
def test_router_split_x_from_7_tokens(ctx, eff, orc, tname, tokens, k, rows, split):
    """From 7 tokens where k > 4096 every type takes the split-x product (the
    16-row GEMV would hold 7-8 tokens' x digits in 97 KB of LDS or more); at
    k = 4096 only Q4_K and Q6_K, and only from 5120 rows; at 6 tokens the
    GEMV stays. Both meet the f64 bar."""
    if split is None:
        split = tname != "Q8_0"
    t, data, gguf, n = make_weights(eff, tname, rows, k, 900 + tokens + k + rows)
    x = eff.fill_normal(901 + tokens, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    after = ctx.stats()
    assert after["split"] - before["split"] == (1 if split else 0)
    check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"router {tname} M={tokens} k={k} rows={rows}")
    for b in (wb, xb, yb):
        b.free()


def test_split_x_k_slices_graph_replays(ctx, eff, orc):
    """A recorded k-sliced split-x product (its preparation and the product,
    64 row tiles in 4 slices) replayed several times, with eager sliced
    products of other shapes between the replays (on the same arrival
    counters): every replay gives the eager bits, which meet the f64 bar."""
    rows, k, tokens = 2048, 8192, 32
    t, data, gguf, n = make_weights(eff, "Q4_K", rows, k, 885)
    x = eff.fill_normal(886, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    y2 = ctx.alloc(tokens * rows * 4)
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    y0 = yb.read(np.uint32)
    check_close(y0.view(np.float32), orc.gemv_f64(orc.Q4_K, gguf, rows, k, x, tokens), "split-x k slices")
    ctx.qmatmul(t, wb, xb, y2, rows // 2, k, 24)     # grows nothing the recording needs
    ctx.graph_begin()
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    g = ctx.graph_end()
    try:
        for r in range(4):
            yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
            g.launch()
            ctx.sync()
            got = yb.read(np.uint32)
            assert np.array_equal(got, y0), f"replay {r}: {np.count_nonzero(got != y0)} outputs differ"
            ctx.qmatmul(t, wb, xb, y2, rows // 2, k, 24)   # another tile count on the same counters
    finally:
        g.destroy()
    for b in (wb, xb, yb, y2):
        b.free()


@pytest.mark.parametrize("tname", ["Q2_K", "IQ2_XXS"])
@pytest.mark.parametrize("tokens,k", [(4, 2304), (8, 2048), (8, 2560), (5, 256)])
def test_split_x_one_launch_bit_identical(ctx, eff, orc, tname, tokens, k, split_from_4):
    """Up to 8 tokens of Q2_K / IQ2_XXS the product prepares x itself (one
    launch, where the rows give 192 workgroups or more and so no k slices, and
    the workgroups times k stay within 256 x 2048);
    the same 32 x 8 plan with the preparation launch (EFF_OPT_SPLIT_CONFIG =
    1) gives the same bits, and both meet the f64 bar (one and two blocks per
    wave, a single block per row)."""
    rows = 6200
    t, data, gguf, n = make_weights(eff, tname, rows, k, 500 + tokens + k)
    x = eff.fill_normal(5000 + tokens + k, 1.0, tokens * k)
    wb, xb = ctx.upload(data), ctx.upload(x)
    got = []
    for cfg in (0, 1):
        yb = ctx.alloc(tokens * rows * 4)
        ctx.set_option(eff.OPT_SPLIT_CONFIG, cfg)
        try:
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
        finally:
            ctx.set_option(eff.OPT_SPLIT_CONFIG, 0)
        got.append(yb.read(np.uint32))
        yb.free()
    assert np.array_equal(got[0], got[1])
    check_close(got[0].view(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"split-x one launch {tname} M={tokens} k={k}")
    wb.free()
    xb.free()


@pytest.mark.parametrize("tname", ["Q2_K", "IQ2_XXS"])
@pytest.mark.parametrize("tokens", [5, 8])
def test_split_x_few_tokens_wide_grid(ctx, eff, orc, tname, tokens, split_from_4):
    """At 5-8 tokens over many rows (32000: 1000 workgroups of 32 rows) the
    product runs 64 rows x 4 waves with x prepared by its own launch, not the
    one-launch product: the forced 64 x 4 plan gives the same bits, the x
    layout answers (no NOT_APPLICABLE), and the f64 bar holds."""
    rows, k = 32000, 512
    t, data, gguf, n = make_weights(eff, tname, rows, k, 520 + tokens)
    x = eff.fill_normal(5200 + tokens, 1.0, tokens * k)
    wb, xb = ctx.upload(data), ctx.upload(x)
    nbytes, lay = ctx.qmatmul_x_layout(t, rows, k, tokens)
    assert lay >= 0x100 and nbytes > 0
    got = []
    for cfg in (0, 2):
        yb = ctx.alloc(tokens * rows * 4)
        ctx.set_option(eff.OPT_SPLIT_CONFIG, cfg)
        try:
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
        finally:
            ctx.set_option(eff.OPT_SPLIT_CONFIG, 0)
        got.append(yb.read(np.uint32))
        yb.free()
    assert np.array_equal(got[0], got[1])
    check_close(got[0].view(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens),
                f"split-x 64 x 4 {tname} M={tokens} rows={rows}")
    wb.free()
    xb.free()


@pytest.mark.parametrize("tname", SPLIT_TYPES)
def test_split_x_dynamic_range_and_non_finite(ctx, eff, orc, tname, split_from_4):
    """x scaled per (token, 256-block): zero, tiny, huge and subnormal values in
    one block, outliers among ordinary values, a whole token at 1e-3; a NaN or an
    infinity makes only its own token's outputs non-finite."""
    rows, k, tokens = 40, 2048, 6
    t, data, gguf, n = make_weights(eff, tname, rows, k, 77)
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (tokens, k)).astype(np.float32)
    x[0, :32] = 0.0
    x[0, 32:64] *= 1e-30
    x[0, 64:96] *= 1e30
    x[1, ::37] *= 1e4
    x[1, 96:128] = np.float32(1e-40)
    x[2, :] *= 1e-3
    x[3, 256:512] = 0.0
    wb, xb, yb = ctx.upload(data), ctx.upload(x.reshape(-1)), ctx.alloc(tokens * rows * 4)
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    check_close(yb.read(np.float32), orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x.reshape(-1), tokens),
                f"split-x {tname} x range")
    x[4, 700] = np.nan
    x[5, 1500] = np.inf
    xb2 = ctx.upload(x.reshape(-1))
    ctx.qmatmul(t, wb, xb2, yb, rows, k, tokens)
    y = yb.read(np.float32).reshape(tokens, rows)
    assert np.all(~np.isfinite(y[4])) and np.all(~np.isfinite(y[5])) and np.all(np.isfinite(y[:4]))
    for b in (wb, xb, xb2, yb):
        b.free()


# ---- router, NOT_APPLICABLE and errors -----------------------------------------------

def test_router_paths_and_stats(ctx, eff, orc):
    rows, k = 96, 512
    t, data, gguf, n = make_weights(eff, "Q4_K", rows, k, 90)
    wb = ctx.upload(data)
    before = ctx.stats()
    for tokens in (1, 5, 9, 33, 64):
        x = eff.fill_normal(91 + tokens, 1.0, tokens * k)
        xb, yb = ctx.upload(x), ctx.alloc(tokens * rows * 4)
        ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
        check_close(yb.read(np.float32), orc.gemv_f64(orc.Q4_K, gguf, rows, k, x, tokens), f"matmul T={tokens}")
    after = ctx.stats()
    # 1..8 tokens count as GEMV calls (the int8 matrix-core GEMVs); Q4_K from 9
    # tokens runs the split-x product at every token count (f32 accuracy, as
    # the reference's generic kernel)
    assert after["gemv"] - before["gemv"] == 2
    assert after["split"] - before["split"] == 3
    assert after["skinny"] == before["skinny"] and after["gemm"] == before["gemm"]
    # Q8_0: the split-x product below 64 tokens, the fp16 GEMM from 64
    t8, data8, gguf8, _ = make_weights(eff, "Q8_0", rows, k, 92)
    w8 = ctx.upload(data8)
    before = ctx.stats()
    for tokens, oracle_fn in ((33, orc.gemv_f64), (64, orc.gemm_f16)):
        x = eff.fill_normal(93 + tokens, 1.0, tokens * k)
        xb, yb = ctx.upload(x), ctx.alloc(tokens * rows * 4)
        ctx.qmatmul(t8, w8, xb, yb, rows, k, tokens)
        check_close(yb.read(np.float32), oracle_fn(orc.Q8_0, gguf8, rows, k, x, tokens), f"matmul Q8_0 T={tokens}")
    after = ctx.stats()
    # 33 tokens: the split-x product (f32-accurate, as the reference's tiled
    # GEMM below DRIFT's threshold); 64: the fp16 GEMM
    assert after["split"] - before["split"] == 1 and after["gemm"] - before["gemm"] == 1
    assert after["skinny"] == before["skinny"]


def test_router_split_x_threshold(ctx, eff, orc):
    """Q2_K: 4 tokens run the int8 matrix-core GEMV, 5 the split-x product, both
    against the f64 oracle; the option moves the threshold and refuses 1..3."""
    rows, k = 96, 512
    t, data, gguf, n = make_weights(eff, "Q2_K", rows, k, 95)
    wb = ctx.upload(data)
    for tokens, low, split in ((4, 0, 0), (5, 0, 1), (7, 8, 0), (4, 4, 1)):
        x = eff.fill_normal(96 + tokens, 1.0, tokens * k)
        xb, yb = ctx.upload(x), ctx.alloc(tokens * rows * 4)
        ctx.set_option(eff.OPT_SPLIT_MIN_TOKENS, low)
        try:
            before = ctx.stats()["split"]
            ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
            assert ctx.stats()["split"] - before == split, (tokens, low)
        finally:
            ctx.set_option(eff.OPT_SPLIT_MIN_TOKENS, 0)
        check_close(yb.read(np.float32), orc.gemv_f64(orc.Q2_K, gguf, rows, k, x, tokens),
                    f"matmul Q2_K T={tokens} split-x from {low or 'default'}")
        xb.free()
        yb.free()
    with pytest.raises(eff.EffError):
        ctx.set_option(eff.OPT_SPLIT_MIN_TOKENS, 3)
    wb.free()


@pytest.mark.parametrize("tokens", [64, 100, 512])
def test_router_q6_k_prefill_is_f32_accurate(ctx, eff, orc, tokens):
    """Q6_K prefill through quant.matmul stays f32-accurate (the reference's
    fp16 GEMMs read Q8_0/Q4_0 only and its Q6_K prefill runs the f32 generic
    kernel, ops.js:117-128): against the f64 oracle, on the split-x product,
    no fp16 GEMM launched."""
    rows, k = 1000, 2048
    t, data, gguf, n = make_weights(eff, "Q6_K", rows, k, 600 + tokens)
    x = eff.fill_normal(601 + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    after = ctx.stats()
    check_close(yb.read(np.float32), orc.gemv_f64(orc.Q6_K, gguf, rows, k, x, tokens), f"matmul Q6_K T={tokens}")
    assert after["gemm"] == before["gemm"]
    assert after["split"] - before["split"] == 1 and after["skinny"] == before["skinny"]
    for b in (wb, xb, yb):
        b.free()


@pytest.mark.parametrize("tname,lote", [("Q8_0", 100), ("Q8_0", 300), ("Q8_0", 1100), ("Q8_0R", 300),
                                        ("Q8_0R", 1100)])
def test_gemm_planned_tail_gives_the_batch_row_bits(ctx, eff, tname, lote):
    """gemm2.cola (ops.gemm2.js:282-303): the last token run alone with the
    batch's plan gives the bits of the batch's last row (128 x 32 tiles at
    100 tokens, 128 x 128 at 300, 256 x 256 / 256 x 128 at 1100); the first
    token too, and a run over the first 3 tokens."""
    rows, k = 272, 1024
    t, data, gguf, n = make_weights(eff, tname, rows, k, 700 + lote)
    x = eff.fill_normal(701 + lote, 1.0, lote * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(lote * rows * 4)
    ctx.qgemm(t, wb, xb, yb, rows, k, lote)
    y = yb.read(np.uint32).reshape(lote, rows)
    x1, y1, y3 = ctx.upload(x[(lote - 1) * k:]), ctx.alloc(rows * 4), ctx.alloc(3 * rows * 4)
    ctx.qgemm_planned(t, wb, x1, y1, rows, k, 1, lote)
    assert np.array_equal(y1.read(np.uint32), y[lote - 1])
    ctx.qgemm_planned(t, wb, xb, y3, rows, k, 3, lote)
    assert np.array_equal(y3.read(np.uint32).reshape(3, rows), y[:3])
    with pytest.raises(eff.NotApplicable):
        ctx.qgemm_planned(t, wb, x1, y1, rows, k, 1, 63)
    with pytest.raises(eff.EffError):
        ctx.qgemm_planned(t, wb, xb, yb, rows, k, lote + 1, lote)
    for b in (wb, xb, yb, x1, y1, y3):
        b.free()


@pytest.mark.parametrize("tname,tokens,lote", [("Q8_0", 300, 300), ("Q8_0", 1100, 1100), ("Q8_0R", 100, 100),
                                               ("Q8_0", 1, 300), ("Q8_0R", 3, 1100)])
def test_gemm_prepared_x_serves_several_products(ctx, eff, tname, tokens, lote):
    """x prepared once (eff_gemm_prepare_x) serves two products over other
    weights (the q / k / v of one activation), each with the bits of
    eff_qgemm_planned over x; one conversion in all; the layout id follows the
    plan, and a call the GEMM does not apply to is NOT_APPLICABLE."""
    k = 1024
    rows = (272, 160)
    ws = [make_weights(eff, tname, r, k, 750 + r + lote) for r in rows]
    x = eff.fill_normal(751 + lote, 1.0, tokens * k)
    xb = ctx.upload(x)
    nbytes, lay = ctx.gemm_x_layout(ws[0][0], rows[0], k, tokens, lote)
    assert (nbytes, lay) == ctx.gemm_x_layout(ws[1][0], rows[1], k, tokens, lote)
    xh = ctx.alloc(nbytes)
    wbs = [upload_w(ctx, eff, tname, data, n) for (t, data, gguf, n) in ws]
    y1s = [ctx.alloc(tokens * r * 4) for r in rows]
    before = ctx.stats()["gemm_x"]
    ctx.gemm_prepare_x(ws[0][0], xb, xh, rows[0], k, tokens, lote)
    for (t, _, _, _), r, wb, y1 in zip(ws, rows, wbs, y1s):
        ctx.qgemm_prepared(t, wb, xh, y1, r, k, tokens, lote)
    assert ctx.stats()["gemm_x"] == before + 1
    for (t, _, _, _), r, wb, y1 in zip(ws, rows, wbs, y1s):
        y2 = ctx.alloc(tokens * r * 4)
        ctx.qgemm_planned(t, wb, xb, y2, r, k, tokens, lote)
        assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32)), (tname, r)
        for b in (wb, y1, y2):
            b.free()
    with pytest.raises(eff.NotApplicable):
        ctx.gemm_x_layout(ws[0][0], rows[0], k, 1, 63)
    with pytest.raises(eff.EffError):
        ctx.gemm_prepare_x(ws[0][0], xb, ctx.alloc(16), rows[0], k, tokens, lote)    # xh too small
    xb.free()
    xh.free()


@pytest.mark.parametrize("tokens", [9, 33, 100])
def test_matmul_prepared_x_serves_several_products(ctx, eff, tokens):
    """The router's x prepared once per layout (eff_qmatmul_prepare_x) serves
    products of every type of that layout and any rows, each with the bits of
    eff_qmatmul over x: IQ2_XXS, Q6_K and Q8_0 share one split-x layout, Q2_K
    and Q4_K have their own (with their group sums), and Q8_0 from the GEMM's
    threshold reads the fp16 GEMM's. One preparation per layout in all."""
    k = 2304
    mats = [("Q2_K", 77), ("Q2_K", 150), ("Q4_K", 96), ("Q4_K", 33), ("IQ2_XXS", 77), ("Q6_K", 64),
            ("Q8_0", 130), ("Q8_0", 40)]
    x = eff.fill_normal(8100 + tokens, 1.0, tokens * k)
    xb = ctx.upload(x)
    groups = {}
    for tname, r in mats:
        nbytes, lay = ctx.qmatmul_x_layout(eff.TYPES[tname], r, k, tokens)
        groups.setdefault(lay, []).append((tname, r, nbytes))
    split = {lay for lay in groups if lay >= 0x100}
    expect = {0x101: {"Q2_K"}, 0x102: {"Q4_K"}, 0x100: {"IQ2_XXS", "Q6_K"} | ({"Q8_0"} if tokens < 64 else set())}
    assert split == set(expect), groups
    for lay in split:
        assert {tname for tname, _, _ in groups[lay]} == expect[lay], (lay, groups[lay])
        assert len({nb for _, _, nb in groups[lay]}) == 1, groups[lay]   # the bytes follow tokens and k only
    assert len(groups) == len(split) + (1 if tokens >= 64 else 0)
    before = ctx.stats()
    for lay, members in groups.items():
        tname0, r0, nbytes = members[0]
        xp = ctx.alloc(max(nb for _, _, nb in members))
        ctx.qmatmul_prepare_x(eff.TYPES[tname0], xb, xp, r0, k, tokens)
        for tname, r, _ in members:
            t, data, _, _ = make_weights(eff, tname, r, k, 8200 + r + tokens)
            wb, y1, y2 = ctx.upload(data), ctx.alloc(tokens * r * 4), ctx.alloc(tokens * r * 4)
            ctx.qmatmul_prepared(t, wb, xp, y1, r, k, tokens)
            ctx.qmatmul(t, wb, xb, y2, r, k, tokens)
            assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32)), (tname, r, tokens, hex(lay))
            for b in (wb, y1, y2):
                b.free()
        xp.free()
    after = ctx.stats()
    n_mats = len(mats)
    n_gemm = len(groups[min(groups)]) if tokens >= 64 else 0
    # one preparation per layout, plus the one of each eff_qmatmul beside it
    assert after["split_x"] - before["split_x"] == len(split) + (n_mats - n_gemm)
    assert after["gemm_x"] - before["gemm_x"] == (1 + n_gemm if tokens >= 64 else 0)
    assert after["split"] - before["split"] == 2 * (n_mats - n_gemm)
    xb.free()


def test_matmul_prepared_x_not_applicable_and_errors(ctx, eff):
    """Calls whose path reads x itself answer NOT_APPLICABLE (the GEMVs, the
    one-launch split-x product up to 8 tokens, the token groups); a forced
    configuration that prepares x (also one with k in two slices) gives
    eff_qmatmul's bits; a short buffer is refused."""
    k = 2304
    # (the one-launch product over 8192 rows: 256 workgroups, no k slices, k = 2048)
    for tname, r, kk, tokens in [("Q2_K", 64, k, 4), ("Q2_K", 8192, 2048, 8), ("IQ2_XXS", 8192, 2048, 5),
                                 ("Q4_K", 64, k, 8), ("Q8_0R", 64, 2080, 33), ("Q8_0", 64, 2080, 33)]:
        with pytest.raises(eff.NotApplicable):
            ctx.qmatmul_x_layout(eff.TYPES[tname], r, kk, tokens)
    t, data, _, _ = make_weights(eff, "Q2_K", 77, k, 8300)
    wb = ctx.upload(data)
    try:
        ctx.set_option(eff.OPT_SPLIT_CONFIG, 3)      # 64 rows x 4 waves, k in two slices
        nbytes, lay = ctx.qmatmul_x_layout(t, 77, k, 33)
        assert lay == 0x101
        x = eff.fill_normal(8302, 1.0, 33 * k)
        xb, xp = ctx.upload(x), ctx.alloc(nbytes)
        y1, y2 = ctx.alloc(33 * 77 * 4), ctx.alloc(33 * 77 * 4)
        ctx.qmatmul_prepare_x(t, xb, xp, 77, k, 33)
        ctx.qmatmul_prepared(t, wb, xp, y1, 77, k, 33)
        ctx.qmatmul(t, wb, xb, y2, 77, k, 33)
        assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32))
        for b in (xb, xp, y1, y2):
            b.free()
        ctx.set_option(eff.OPT_SPLIT_CONFIG, 1)      # 32 rows x 8 waves, x prepared, at 8 tokens
        nbytes, lay = ctx.qmatmul_x_layout(t, 77, k, 8)
        assert lay == 0x101
        x = eff.fill_normal(8301, 1.0, 8 * k)
        xb, xp = ctx.upload(x), ctx.alloc(nbytes)
        y1, y2 = ctx.alloc(8 * 77 * 4), ctx.alloc(8 * 77 * 4)
        ctx.qmatmul_prepare_x(t, xb, xp, 77, k, 8)
        ctx.qmatmul_prepared(t, wb, xp, y1, 77, k, 8)
        ctx.qmatmul(t, wb, xb, y2, 77, k, 8)
        assert np.array_equal(y1.read(np.uint32), y2.read(np.uint32))
        small = ctx.alloc(64)
        with pytest.raises(eff.EffError):
            ctx.qmatmul_prepared(t, wb, small, y1, 77, k, 8)                    # xp too small
        with pytest.raises(eff.EffError):
            ctx.qmatmul_prepare_x(t, xb, xp, 77, k, 9)                          # x too small
        for b in (xb, xp, y1, y2, small):
            b.free()
    finally:
        ctx.set_option(eff.OPT_SPLIT_CONFIG, 0)
        wb.free()


# ---- the reference CPU path's arithmetic (eff_qmatmul_cpu_path) ----------------------------

@pytest.mark.parametrize("rows,k,tokens", [(77, 32, 1), (300, 2080, 3), (64, 4096, 65), (130, 2048, 7),
                                           (33, 256, 130), (77, 2080, 40), (33, 96, 16)])
def test_cpu_path_product_bit_exact(ctx, eff, orc, rows, k, tokens):
    """The CPU path's arithmetic on the GPU gives the bits of the oracle's
    restatement of it (or_cpu_matmul: 8-bit x blocks, int32 block dots, the
    f32 terms added in block order), below 16 tokens (a wave per row) and
    from 16 (the block dots on the matrix cores, 8-block chunks staged in
    LDS): more than 64 blocks per row, more than 64 tokens (two and three
    token chunks), block counts that are not multiples of 64 or of 8 (a last
    chunk of one block; 3 blocks in all), rows and tokens that do not fill
    the last workgroup."""
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 1200 + rows + k + tokens)
    x = eff.fill_normal(1300 + rows + tokens, 1.0, tokens * k)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    before = ctx.stats()["cpu_path"]
    ctx.qmatmul_cpu_path(t, wb, xb, yb, rows, k, tokens)
    assert ctx.stats()["cpu_path"] == before + 1
    ref = orc.cpu_matmul(orc.Q8_0, gguf, rows, k, x, tokens, 4)
    got = yb.read(np.float32, tokens * rows).reshape(tokens, rows)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
        f"{int(np.sum(got.view(np.uint32) != ref.view(np.uint32)))} outputs differ"
    for b in (wb, xb, yb):
        b.free()


def test_cpu_path_product_edge_blocks(ctx, eff, orc):
    """Blocks whose quantization the CPU path's rounding decides: ties at
    x / d = n + 1/2 in both signs (max |x| = 127 and 63.5, so 1 / d is exact),
    an all-zero block (d = 0: zero quants, zero term), one value per block,
    large and small magnitudes; bit-equal to the restatement, whose block
    fields are checked here too."""
    rows, k, tokens = 40, 256, 4
    x = np.zeros((tokens, k), np.float32)
    x[0, :32] = [127.0] + [v + 0.5 for v in range(-15, 16)]
    x[0, 32:64] = [63.5] + [(v + 0.5) / 2 for v in range(-15, 16)]
    x[1, 64] = -3.0e5                         # one value in its block
    x[1, 96:128] = np.linspace(-1e-30, 1e-30, 32, dtype=np.float32)
    x[2] = eff.fill_normal(1401, 1.0, k)
    x[3] = eff.fill_normal(1402, 1e4, k)
    x = x.reshape(-1)
    acts = orc.cpu_quantize_acts(x, k, tokens)
    assert acts[0]["d"] == 1.0 and list(acts[0]["q"][1:4]) == [-15, -14, -13]   # -14.5 -> -15, -13.5 -> -14
    assert acts[0]["q"][16] == 1 and acts[0]["q"][15] == -1                       # 0.5 -> 1, -0.5 -> -1
    assert acts[1]["d"] == 0.5 and acts[1]["q"][16] == 1
    assert acts[8]["d"] == 0.0 and not acts[8]["q"].any()                        # an all-zero block
    assert acts[10]["q"][0] == -127 and not acts[10]["q"][1:].any()              # one value in its block
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 1403)
    wb, xb, yb = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qmatmul_cpu_path(t, wb, xb, yb, rows, k, tokens)
    ref = orc.cpu_matmul(orc.Q8_0, gguf, rows, k, x, tokens, 2)
    assert np.array_equal(yb.read(np.uint32, tokens * rows), ref.view(np.uint32).reshape(-1))
    for b in (wb, xb, yb):
        b.free()


def test_cpu_path_product_gap_and_errors(ctx, eff, orc):
    """Against the f64 product the CPU path's 8-bit activations cost about
    5e-3 relative L2, the gap the default router does not have; other types
    are NOT_APPLICABLE (its kernels are Q8_0 and Q4_0), k not a multiple of
    32 is a shape error."""
    rows, k, tokens = 256, 2048, 2
    t, data, gguf, n = make_weights(eff, "Q8_0", rows, k, 1500)
    x = eff.fill_normal(1501, 1.0, tokens * k)
    wb, xb, y1, y2 = ctx.upload(data), ctx.upload(x), ctx.alloc(tokens * rows * 4), ctx.alloc(tokens * rows * 4)
    ctx.qmatmul_cpu_path(t, wb, xb, y1, rows, k, tokens)
    ctx.qmatmul(t, wb, xb, y2, rows, k, tokens)
    ref = orc.gemv_f64(orc.Q8_0, gguf, rows, k, x, tokens)
    gap = np.linalg.norm(y1.read(np.float32).reshape(ref.shape) - ref) / np.linalg.norm(ref)
    acc = np.linalg.norm(y2.read(np.float32).reshape(ref.shape) - ref) / np.linalg.norm(ref)
    print(f"cpu path against f64: {gap:.2e}; default router: {acc:.2e}", flush=True)
    assert 1e-3 < gap < 2e-2 and acc < 1e-5
    t4, data4, _, _ = make_weights(eff, "Q4_K", rows, k, 1502)
    w4 = ctx.upload(data4)
    with pytest.raises(eff.NotApplicable):
        ctx.qmatmul_cpu_path(t4, w4, xb, y1, rows, k, tokens)
    with pytest.raises(eff.EffError):
        ctx.qmatmul_cpu_path(t, wb, xb, y1, rows, 48, tokens)
    for b in (wb, xb, y1, y2, w4):
        b.free()


def test_read_ticket_snapshots_at_begin(ctx, eff):
    """eff_read_begin enqueues the copy at once: a write enqueued after it is
    not in the snapshot; the buffer can be reused right away."""
    a = np.arange(4096, dtype=np.uint32)
    b = ctx.upload(a)
    fin = ctx.read_async(b, np.uint32)
    b.write(a[::-1].copy())
    assert np.array_equal(fin(), a)
    assert np.array_equal(b.read(np.uint32), a[::-1])
    # 600 writes of 16 KiB go through the 8 MiB staging ring (wrapping once);
    # each lands in order
    c = ctx.alloc(4 * 16384)
    for i in range(600):
        c.write(np.full(4096, i, np.uint32), offset=16384 * (i % 4))
    got = c.read(np.uint32).reshape(4, 4096)
    for j in range(4):
        assert np.all(got[j] == 596 + j)
    b.free()
    c.free()


def test_not_applicable_and_errors(ctx, eff):
    rows, k = 8, 256
    t, data, gguf, n = make_weights(eff, "Q4_K", rows, k, 1)
    wb, xb, yb = ctx.upload(data), ctx.alloc(64 * k * 4), ctx.alloc(64 * rows * 4)
    with pytest.raises(eff.NotApplicable):
        ctx.qgemv(t, wb, xb, yb, rows, k, 9)
    with pytest.raises(eff.NotApplicable):
        ctx.qgemm(t, wb, xb, yb, rows, k, 32)
    with pytest.raises(eff.EffError) as e:
        ctx.qmatmul(t, wb, xb, yb, rows, 300, 1)
    assert e.value.code == eff.E_SHAPE and "300" in str(e.value)
    with pytest.raises(eff.EffError) as e:
        ctx.qmatmul(99, wb, xb, yb, rows, k, 1)
    assert e.value.code == eff.E_TYPE
    for shape in ((0, k, 1), (rows, 0, 1), (rows, k, 0)):   # empty shapes are refused, nothing launched
        with pytest.raises(eff.EffError) as e:
            ctx.qmatmul(t, wb, xb, yb, *shape)
        assert e.value.code == eff.E_INVALID and "empty" in str(e.value)
    with pytest.raises(eff.EffError) as e:
        ctx.qmatmul(t, wb, xb, yb, rows * 4, k, 1)      # W too small for the call
    assert e.value.code == eff.E_BOUNDS
    # Q8_0R: unmarked buffer, and a call beyond the marked tensor
    _, data_r, _, nr = make_weights(eff, "Q8_0R", rows, k, 2)
    rb = ctx.upload(data_r)
    with pytest.raises(eff.EffError) as e:
        ctx.qmatmul(eff.Q8_0R, rb, xb, yb, rows, k, 1)
    assert e.value.code == eff.E_MARK
    rb.mark_r(nr)
    assert rb.blocks_r() == nr
    ctx.qmatmul(eff.Q8_0R, rb, xb, yb, rows, k, 1)
    with pytest.raises(eff.EffError) as e:
        ctx.qmatmul(eff.Q8_0R, rb, xb, yb, rows + 1, k, 1)
    assert e.value.code == eff.E_MARK
    with pytest.raises(eff.EffError):
        ctx.alloc(1000).mark_r(64)                      # wrong size for 64 blocks
    # options
    ctx.set_option(eff.OPT_GEMM_MIN_TOKENS, 16)
    try:
        ctx.qgemm(t, wb, xb, yb, rows, k, 32)
    finally:
        ctx.set_option(eff.OPT_GEMM_MIN_TOKENS, 64)
    with pytest.raises(eff.EffError):
        ctx.set_option(eff.OPT_GEMV_MAX_TOKENS, 9)


# ---- top-k ---------------------------------------------------------------------------

def run_topk(ctx, eff, vals, m, base=0, penal=(), serial=7):
    buf = np.zeros(base + vals.size, np.float32)
    buf[base:] = vals
    lb = ctx.upload(buf)
    out = ctx.topk(lb, base, vals.size, m, penal, serial)
    return eff.parse_topk(out.read(np.uint32))


@pytest.mark.parametrize("vocab,m", [(1, 1), (100, 40), (4096, 40), (4097, 40), (65536, 40), (65536, 100),
                                     (65536, 192), (70000, 192), (10, 40), (200000, 7), (63, 40), (65, 40),
                                     (257, 192), (1 << 20, 100), (65537, 40)])
def test_topk_bit_exact(ctx, eff, orc, vocab, m):
    rng = np.random.default_rng(vocab + m)
    vals = rng.normal(0, 3, vocab).astype(np.float32)
    vals[rng.integers(0, vocab, max(1, vocab // 8))] = 2.5      # ties, broken by index
    if vocab > 3:
        vals[1], vals[2] = -0.0, 0.0
    r = run_topk(ctx, eff, vals, m, base=3, penal=[0, vocab - 1, vocab + 5], serial=42)
    ids, bits, nan = orc.topk(vals.view(np.uint32), m)
    assert r["n"] == len(ids) and r["flags"] == 0 and r["serial"] == 42
    assert r["chunks"] == (vocab + 4095) // 4096
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["bits"], bits)
    assert np.array_equal(r["penal_bits"], np.array([vals.view(np.uint32)[0], vals.view(np.uint32)[-1], 0], np.uint32))


def test_topk_flags_nan_and_limits(ctx, eff):
    vals = np.arange(5000, dtype=np.float32)
    vals[1234] = np.nan
    r = run_topk(ctx, eff, vals, 40)
    assert r["flags"] & 2
    lb = ctx.upload(vals)
    with pytest.raises(eff.NotApplicable):
        ctx.topk(lb, 0, vals.size, 193)
    with pytest.raises(eff.NotApplicable):
        ctx.topk(lb, 0, vals.size, 40, penal_ids=list(range(129)))


@pytest.mark.parametrize("layout", ["periodic", "ascending", "descending", "two_levels"])
def test_topk_layouts(ctx, eff, orc, layout):
    """Layouts against the per-thread-maximum threshold of the select: "periodic"
    puts the large logits on 48 of every 256 positions, so each chunk keeps 768
    composites above its threshold and takes the radix fallback; sorted inputs
    put a chunk's largest logits on one stride."""
    rng = np.random.default_rng(5)
    vocab, m = 65536, 48
    j = np.arange(vocab)
    if layout == "periodic":
        vals = np.where(j % 256 < 48, 10.0, 0.0) + rng.normal(0, 1, vocab)
    elif layout == "ascending":
        vals = j * 1e-3
    elif layout == "descending":
        vals = -j * 1e-3
    else:
        vals = np.where(rng.random(vocab) < 0.01, 5.0, -5.0)
    vals = vals.astype(np.float32)
    r = run_topk(ctx, eff, vals, m)
    ids, bits, nan = orc.topk(vals.view(np.uint32), m)
    assert r["n"] == len(ids) and r["flags"] == 0
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["bits"], bits)


@pytest.mark.parametrize("vocab,m", [(65536, 192), (3000001, 150)])
def test_topk_clustered_in_one_group(ctx, eff, orc, vocab, m):
    """All the largest logits inside one group of consecutive logits (64 at
    vocab 65536, 64 * 46 at 3,000,001): the group's 4-element list is
    saturated and the select reads the group whole."""
    rng = np.random.default_rng(vocab)
    vals = rng.normal(0, 1, vocab).astype(np.float32)
    gs = 64 * ((vocab + 65535) // 65536)
    g0 = (vocab // gs // 2) * gs
    vals[g0:g0 + gs] = 50.0 + rng.normal(0, 1, gs).astype(np.float32)
    vals[g0 + 7] = vals[g0 + 9]                                 # a tie inside the group
    r = run_topk(ctx, eff, vals, m)
    ids, bits, nan = orc.topk(vals.view(np.uint32), m)
    assert r["n"] == len(ids) and r["flags"] == 0
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["bits"], bits)


@pytest.mark.parametrize("tname,rows,k,m,cluster", [
    ("Q6_K", 65536, 2048, 40, 0),          # the C4 head: records from the GEMV, 512 groups of 3 or 5 tiles
    ("Q6_K", 40001, 2048, 192, 5000),      # ragged rows; the largest logits in 5 tiles of 32 rows
    ("Q6_K", 65536, 2048, 40, 60000),      # ... in tiles the second half of the grid takes last (its 5th)
    ("Q6_K", 65664, 512, 100, 5000),       # 513 groups of 4 tiles (an even grid: 514)
    ("Q6_K", 65536, 512, 40, 5000),        # the wave-maximum threshold, then saturated groups read whole
    ("Q6_K", 40000, 2304, 40, 0),          # an odd block count per row (per-row load offsets)
    ("Q6_K", 131072, 512, 64, 0),          # 1024 groups, the most one selection holds (two per thread)
    ("Q6_K", 131073, 512, 40, 0),          # more groups than one selection holds: GEMV, then eff_topk
    ("Q6_K", 65536, 1024, 40, 0),          # 4 k slices per row group (k of 4 to 7 blocks)
    ("Q6_K", 65536, 1280, 100, 30000),     # ... with an odd block count
    ("Q8_0", 50000, 512, 40, 0),           # no row kernel: GEMV, then eff_topk
])
def test_qgemv_topk_equals_gemv_then_topk(ctx, eff, orc, tname, rows, k, m, cluster):
    """eff_qgemv_topk gives the logits and the top-k record of eff_qmatmul
    followed by eff_topk, bit for bit, and the record is the oracle's top-m of
    those logits."""
    base = "Q8_0" if tname == "Q8_0R" else tname
    wf = eff.fill_normal(rows % 1000 + 1011, 0.02, rows * k).reshape(rows, k)
    if cluster:
        wf[cluster:cluster + 128] *= 40.0                  # these rows dominate
    w = eff.quantize(base, wf)
    x = eff.fill_normal(12, 1.0, k)
    t = eff.TYPES[tname]
    wb, xb, y1, y2 = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 4), ctx.alloc(rows * 4)
    pen = [3, rows - 1]
    o1 = ctx.qgemv_topk(t, wb, xb, y1, rows, k, m, pen, serial=5)
    ctx.qmatmul(t, wb, xb, y2, rows, k, 1)
    o2 = ctx.topk(y2, 0, rows, m, pen, serial=5)
    ya, yb_ = y1.read(np.uint32), y2.read(np.uint32)
    assert np.array_equal(ya, yb_)
    ra, rb = o1.read(np.uint32), o2.read(np.uint32)
    assert np.array_equal(ra, rb)
    r = eff.parse_topk(ra)
    ids, bits, nan = orc.topk(ya, m)
    assert r["n"] == m and r["flags"] == 0 and r["serial"] == 5
    assert np.array_equal(r["ids"], ids) and np.array_equal(r["bits"], bits)
    if cluster:   # the boosted rows hold the largest logits
        assert np.all((r["ids"][:32] >= cluster) & (r["ids"][:32] < cluster + 128))
    # a call the top-k does not apply to enqueues nothing
    y1.write(np.zeros(rows, np.uint32))
    with pytest.raises(eff.NotApplicable):
        ctx.qgemv_topk(t, wb, xb, y1, rows, k, eff.TOPK_M_MAX + 1)
    assert not np.any(y1.read(np.uint32))
    for b in (wb, xb, y1, y2, o1, o2):
        b.free()


def test_qgemv_topk_nan_in_x(ctx, eff, orc):
    """A NaN in x makes every logit of the head NaN: the record from the GEMV's
    group records equals eff_topk over the same logits bit for bit, NaN flag set."""
    rows, k, m = 65536, 512, 40
    w = eff.quantize("Q6_K", eff.fill_normal(21, 0.02, rows * k))
    x = eff.fill_normal(22, 1.0, k)
    x[100] = np.nan
    t = eff.TYPES["Q6_K"]
    wb, xb, y1 = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 4)
    o1 = ctx.qgemv_topk(t, wb, xb, y1, rows, k, m, [], serial=9)
    o2 = ctx.topk(y1, 0, rows, m, [], serial=9)
    assert np.all(np.isnan(y1.read(np.float32)))
    ra, rb = o1.read(np.uint32), o2.read(np.uint32)
    assert np.array_equal(ra, rb)
    assert eff.parse_topk(ra)["flags"] & 2
    for b in (wb, xb, y1, o1, o2):
        b.free()


def test_topk_all_equal(ctx, eff):
    vals = np.full(9000, 1.5, np.float32)
    r = run_topk(ctx, eff, vals, 40)
    assert list(r["ids"]) == list(range(40))


def test_read_floor_reads_and_checks_its_arguments(ctx, eff):
    """eff_read_floor (the bench's streaming-read floor): every grid shape runs
    over a buffer whose size is not a multiple of any chunk and leaves the sink
    untouched (the XOR of the bytes is not its constant); bad shapes are refused."""
    src = ctx.upload(np.arange(3 * 1024 * 1024 + 48, dtype=np.uint8))
    sink = ctx.upload(np.zeros(4096, np.uint32))
    for wg, un in ((2048, 1), (1024, 2), (1024, 4), (1, 4), (3, 1)):
        ctx.read_floor(src, src.size - 16, wg, un, sink)
    ctx.sync()
    assert not sink.read(np.uint32).any()
    for args, code in (((src.size + 1, 16, 1), eff.E_BOUNDS), ((1024, 16, 3), eff.E_INVALID),
                       ((1024, 0, 1), eff.E_INVALID), ((1024, 8192, 1), eff.E_BOUNDS), ((0, 16, 1), eff.E_INVALID)):
        with pytest.raises(eff.EffError) as e:
            ctx.read_floor(src, args[0], args[1], args[2], sink)
        assert e.value.code == code, args
    src.free()
    sink.free()


# ---- router over seeded random shapes -----------------------------------------------------

def _random_router_cases(n, seed=20261202):
    rng = np.random.default_rng(seed)
    types = ["Q8_0", "Q8_0R", "Q4_K", "Q6_K", "Q2_K", "IQ2_XXS"]
    ks_256 = [256, 512, 768, 1280, 2304, 4096, 8448, 14336, 16384]
    ks_32 = [32, 96, 544, 2080]
    # (at least 3 rows: the bar's max |d| / ||row|| over a single output is its own relative error,
    # which an f32-accurate sum need not keep below 1e-3 where the output cancels to near zero)
    rows_l = [3, 7, 33, 100, 257, 600, 1500, 2048, 3000]
    toks_l = [1, 2, 3, 4, 5, 6, 8, 9, 16, 33, 63, 64, 65, 100, 129, 200, 300]
    cases = []
    while len(cases) < n:
        tname = types[rng.integers(len(types))]
        kl = ks_256 + (ks_32 if tname in ("Q8_0", "Q8_0R") else [])
        k, rows, tokens = kl[rng.integers(len(kl))], rows_l[rng.integers(len(rows_l))], toks_l[rng.integers(len(toks_l))]
        if rows * k * tokens <= 40_000_000:
            cases.append((tname, rows, k, tokens))
    return cases


@pytest.mark.parametrize("case", range(60))
def test_router_random_shapes(ctx, eff, orc, case):
    """60 seeded random (type, rows, k, tokens) through eff_qmatmul, whatever
    path the router takes (the GEMVs, the token groups, the split-x product
    with or without k slices, the fp16 GEMM with or without them): each meets
    its oracle (the fp16-rounded one for Q8_0/Q8_0R from the GEMM's 64
    tokens, f64 otherwise), and a second call gives the same bits."""
    tname, rows, k, tokens = _random_router_cases(60)[case]
    t, data, gguf, n = make_weights(eff, tname, rows, k, 3000 + case)
    x = eff.fill_normal(3100 + case, 1.0, tokens * k)
    wb, xb, yb = upload_w(ctx, eff, tname, data, n), ctx.upload(x), ctx.alloc(tokens * rows * 4)
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    y0 = yb.read(np.uint32)
    if tname in ("Q8_0", "Q8_0R") and tokens >= 64:
        ref = orc.gemm_f16(orc.Q8_0, gguf, rows, k, x, tokens)
    else:
        ref = orc.gemv_f64(oracle_type(orc, tname), gguf, rows, k, x, tokens)
    check_close(y0.view(np.float32), ref, f"router {tname} rows={rows} k={k} M={tokens}")
    yb.write(np.full(tokens * rows, 0x7FC00000, np.uint32))
    ctx.qmatmul(t, wb, xb, yb, rows, k, tokens)
    assert np.array_equal(yb.read(np.uint32), y0)
    for b in (wb, xb, yb):
        b.free()

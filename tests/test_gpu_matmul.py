"""GPU parity: f32 matmul on MFMA vs rayon_matmul restated (oracle).

Tolerance (matmul, BASELINE): |g - c| <= atol + 2e-3 |c| with atol
= 1e-4 * max|c|, i.e. a relative bound on the output scale for entries that
cancel to ~0 (C entries are sums of K products of either sign).  Both sides
accumulate in f32; only the summation order differs.
"""
import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


def check(got, want, what):
    atol = 1e-4 * float(np.abs(want).max() or 1.0)
    assert_close(got, want, 2e-3, atol, what)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (64, 784, 128), (64, 128, 10),
                                   (130, 17, 129), (257, 64, 255), (128, 128, 128),
                                   (256, 512, 384), (31, 4096, 96), (2, 3, 4)])
def test_matmul_shapes(hip, m, k, n):
    g = rng(m * 7 + k * 3 + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    got = hip.matmul(hip.tensor(a), hip.tensor(b))
    assert got.shape == (m, n)
    check(got.numpy(), oracle.matmul(a, b), f"matmul {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [(2048, 1024, 2176), (1152, 2048, 3968), (2047, 1040, 2052)])
def test_matmul_split_k_between_one_and_two_tiles_per_cu(hip, m, k, n):
    """128x128 tiles numbering between one and two per CU with K >= 1024
    (272, 279 and 272 tiles on 256 CUs) are split over K so that a CU gets
    about two workgroups; the splits are summed in a fixed order, so a
    repeated call gives the same bits."""
    g = rng(m + 3 * k + 7 * n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    check(got, oracle.matmul(a, b), f"split {m}x{k}x{n}")
    assert np.array_equal(hip.matmul(ta, tb).numpy(), got)


def test_matmul_leading_dims_and_errors(hip):
    g = rng(5)
    a = g.standard_normal((2, 3, 5)).astype(np.float32)
    b = g.standard_normal((5, 4)).astype(np.float32)
    got = hip.matmul(hip.tensor(a), hip.tensor(b))
    assert got.shape == (2, 3, 4)
    check(got.numpy(), oracle.matmul(a, b), "leading dims")
    with pytest.raises(hip.CloveError):
        hip.matmul(hip.tensor(a), hip.tensor(np.ones((4, 4), np.float32)))


def test_matmul_identity_is_exact(hip):
    a = rng(6).standard_normal((192, 256)).astype(np.float32)
    got = hip.matmul(hip.tensor(a), hip.tensor(np.eye(256, dtype=np.float32))).numpy()
    assert np.array_equal(got, a)


def test_config4_full(hip):
    """Config 4: C = A.B at M=N=K=4096 and the skinny M=32 case, A and B
    normal(0, 1/sqrt(K)), seed 3.  Every element of both products is checked
    against the oracle (rayon_matmul restated: a few seconds on the host's
    cores for the square one), and the square one also against float64."""
    g = rng(3)
    K = 4096
    a = g.normal(0, 1 / np.sqrt(K), (4096, K)).astype(np.float32)
    b = g.normal(0, 1 / np.sqrt(K), (K, 4096)).astype(np.float32)
    tb = hip.tensor(b)
    got = hip.matmul(hip.tensor(a), tb).numpy()
    check(got, oracle.matmul(a, b), "4096^3")
    # float64 with a bound of a few ulps of the K-term sum's scale
    ref64 = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(got - ref64)) < 1e-5
    a32 = a[:32].copy()
    check(hip.matmul(hip.tensor(a32), tb).numpy(), oracle.matmul(a32, b), "skinny 32x4096x4096")


# The strip path (M <= 32, even N, K % 4 == 0): one launch, a workgroup per
# 16-row half of a 32-column strip over the whole K.  The plan takes it only
# when CLOVE_GEMM_STRIP forces it (with B cold in HBM the skinny kernel is
# faster), as on the edge shapes here: K equal to the unrolled walk (256,
# 4096, 16384) or not (k past K masked), partial strips (N % 32 != 0), one or
# two row halves, partial halves.
@pytest.mark.parametrize("m,k,n", [(1, 4, 2), (5, 12, 34), (16, 256, 64), (17, 300, 96),
                                   (31, 2052, 130), (32, 4096, 512), (32, 256, 2),
                                   (20, 16384, 64), (32, 4104, 94), (9, 8188, 4098),
                                   (32, 1024, 4096)])
def test_strip_shapes(hip, monkeypatch, m, k, n):
    monkeypatch.setenv("CLOVE_GEMM_STRIP", "1")
    g = rng(m * 13 + k * 3 + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    check(got, oracle.matmul(a, b), f"strip {m}x{k}x{n}")
    # deterministic: the same plan gives the same bits
    assert np.array_equal(hip.matmul(ta, tb).numpy(), got)


# The skinny path (M <= 64, K % 4 == 0, 16-byte aligned A and B): 32*nb columns
# per workgroup, a K split over the workgroup's waves and across workgroups.
# The plan picks it for B >= 4 MiB; CLOVE_GEMM_SKINNY forces it on the small
# edge shapes here; N % 4 != 0 (N = 1, 33, 31, 5003, 4099, 8191) narrows the
# column blocks per wave.
@pytest.mark.parametrize("m,k,n", [(1, 4, 1), (5, 12, 33), (31, 20, 100), (32, 4096, 96),
                                   (33, 784, 128), (63, 1028, 200), (64, 4100, 64),
                                   (17, 8, 31), (64, 784, 10), (48, 2052, 40), (32, 36, 4096),
                                   (30, 4096, 1000), (64, 2048, 1536), (16, 4096, 5003),
                                   (40, 2048, 4099), (1, 4096, 8191)])
def test_skinny_shapes(hip, monkeypatch, m, k, n):
    monkeypatch.setenv("CLOVE_GEMM_SKINNY", "0")
    g = rng(m * 11 + k * 5 + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    check(hip.matmul(hip.tensor(a), hip.tensor(b)).numpy(), oracle.matmul(a, b),
          f"skinny {m}x{k}x{n}")


@pytest.mark.parametrize("m", [24, 40])
@pytest.mark.parametrize("plan", ["4,1", "2,1", "1,2", "4,5", "2,7", "1,64", "4,64"])
def test_skinny_plan_variants(hip, monkeypatch, m, plan):
    """Every (column blocks per wave, K splits) choice of the skinny plan,
    and the tiled path (CLOVE_GEMM_CFG), computes the same product within
    the matmul bound; each plan is deterministic."""
    g = rng(21 + m)
    k, n = 3076, 72
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    want = oracle.matmul(a, b)
    ta, tb = hip.tensor(a), hip.tensor(b)
    monkeypatch.setenv("CLOVE_GEMM_SKINNY", plan)
    got = hip.matmul(ta, tb).numpy()
    check(got, want, f"skinny plan {plan}")
    assert np.array_equal(got, hip.matmul(ta, tb).numpy())
    monkeypatch.delenv("CLOVE_GEMM_SKINNY")
    monkeypatch.setenv("CLOVE_GEMM_CFG", "1")
    check(hip.matmul(ta, tb).numpy(), want, "tiled path")


def test_skinny_misaligned_a_falls_back(hip):
    """A borrowed A that is not 16-byte aligned takes the tiled path (the
    skinny kernel reads A in 16-byte vectors)."""
    g = rng(22)
    m, k, n = 16, 64, 48
    a = g.normal(0, 1, (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    buf = hip.tensor(np.concatenate([[0.0], a.ravel()]).astype(np.float32))
    av = hip.wrap(buf.device_ptr + 4, (m, k))
    check(hip.matmul(av, hip.tensor(b)).numpy(), oracle.matmul(a, b), "misaligned A")
    del av


# The small path (16 x 16 tiles that cannot fill the chip, K <= 1024,
# K % 4 == 0, 16-byte aligned A): one workgroup per tile, K split over
# 2/4/8/16 waves inside it, partials summed in LDS in wave order.
@pytest.mark.parametrize("m,k,n", [(1, 4, 1), (5, 8, 3), (33, 64, 65), (64, 128, 10),
                                   (31, 200, 100), (64, 256, 64), (100, 500, 33),
                                   (64, 784, 128), (96, 1024, 96), (250, 300, 250)])
def test_small_path_shapes(hip, m, k, n):
    g = rng(31 * m + k + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    check(got, oracle.matmul(a, b), f"small {m}x{k}x{n}")
    assert np.array_equal(got, hip.matmul(ta, tb).numpy()), "small path is deterministic"


@pytest.mark.parametrize("cfg", ["0", "1", "2"])
def test_tiled_split_k_still_covered(hip, monkeypatch, cfg):
    """Shapes the small path now takes, forced through the tiled split-K
    kernels (CLOVE_GEMM_CFG turns the small path off), keep the same product
    within the matmul bound."""
    monkeypatch.setenv("CLOVE_GEMM_CFG", cfg)
    for m, k, n in ((64, 784, 128), (64, 128, 10), (33, 64, 65)):
        g = rng(41 * m + k + n)
        a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
        b = g.normal(0, 1, (k, n)).astype(np.float32)
        check(hip.matmul(hip.tensor(a), hip.tensor(b)).numpy(), oracle.matmul(a, b),
              f"tiled cfg {cfg} {m}x{k}x{n}")


def test_small_path_misaligned_a_falls_back(hip):
    g = rng(23)
    m, k, n = 40, 128, 72
    a = g.normal(0, 1, (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    buf = hip.tensor(np.concatenate([[0.0], a.ravel()]).astype(np.float32))
    av = hip.wrap(buf.device_ptr + 4, (m, k))
    check(hip.matmul(av, hip.tensor(b)).numpy(), oracle.matmul(a, b), "misaligned A")
    del av


@pytest.mark.parametrize("m,k,n", [(0, 5, 7), (5, 7, 0), (0, 0, 0), (5, 0, 7), (1, 0, 1)])
def test_matmul_empty_dimensions(hip, m, k, n):
    """Any zero dimension: the plan has nothing to tile (it used to divide by
    the tile count), and K = 0 gives a zero product."""
    a = np.zeros((m, k), np.float32)
    b = np.zeros((k, n), np.float32)
    got = hip.matmul(hip.tensor(a), hip.tensor(b)).numpy()
    assert got.shape == (m, n) and np.all(got == 0)


# Interior tiles of the 128 x 256, 128 x 128 and 64 x 128 configurations run the
# DMA-staged kernel (slabs moved by buffer->LDS loads); CLOVE_GEMM_DMA=0 runs
# the register-staged kernel.  Same tiles, waves and MFMA order: the same
# bits, single launch and split-K, and both within the matmul bound of the
# oracle.  CLOVE_GEMM_CFG picks the configuration (2: 128 x 128, 5: 128 x 256,
# 6: 64 x 128).
@pytest.mark.parametrize("cfg,m,k,n", [(5, 256, 512, 512), (5, 128, 4096, 256),
                                       (2, 384, 1040, 256), (2, 128, 16, 128),
                                       (2, 256, 8192, 256), (5, 512, 2048, 768),
                                       (6, 64, 8192, 4096), (6, 128, 2048, 256)])
def test_dma_kernel_matches_register_staged(hip, monkeypatch, cfg, m, k, n):
    monkeypatch.setenv("CLOVE_GEMM_CFG", str(cfg))
    g = rng(cfg * 7 + m + k + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    dma = hip.matmul(ta, tb).numpy()
    monkeypatch.setenv("CLOVE_GEMM_DMA", "0")
    staged = hip.matmul(ta, tb).numpy()
    assert np.array_equal(dma, staged)
    check(dma, oracle.matmul(a, b), f"dma cfg {cfg} {m}x{k}x{n}")


@pytest.mark.parametrize("cfg", [2, 5])
def test_dma_kernel_epilogue(hip, monkeypatch, cfg):
    """The fused bias + GELU epilogue on the DMA-staged kernel: the eager
    composition's bits."""
    monkeypatch.setenv("CLOVE_GEMM_CFG", str(cfg))
    g = rng(60 + cfg)
    m, k, n = 256, 1024, 512
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = g.normal(0, 1, (k, n)).astype(np.float32)
    b = g.normal(0, 1, n).astype(np.float32)
    gr = hip.Graph()
    x, wi, bi = gr.input(f"{m},{k}"), gr.input(f"{k},{n}"), gr.input(f"{n}")
    y = gr.op("gelu", gr.op("add", gr.op("matmul", x, wi), bi))
    (fused,) = gr.compile([y]).execute([hip.tensor(a), hip.tensor(w), hip.tensor(b)])
    eager = hip.gelu(hip.add(hip.matmul(hip.tensor(a), hip.tensor(w)), hip.tensor(b)))
    assert np.array_equal(fused.numpy(), eager.numpy())


# Tiles reaching past M or N, or K ending inside the last slab, run the
# DMA-staged kernel too when N % 4 == K % 4 == 0 (rows of A past M, columns
# of B past N and pieces past K read as zeros, stores bounds-checked): the
# register-staged kernel's bits, single launch and split-K (the K tail in
# the last split), plain and with the fused column-bias epilogue.
# N % 4 != 0 or K % 4 != 0 (the last eight, 128x128 and 64x128 tiles) moves
# that operand one float a lane, with the masks per element: the same bits.
@pytest.mark.parametrize("cfg,m,k,n", [(5, 300, 512, 516), (2, 129, 1040, 132),
                                       (2, 200, 8192, 260), (5, 1000, 64, 1100),
                                       (5, 4097, 256, 4096), (2, 130, 4096, 1000),
                                       (5, 257, 4096, 4), (2, 1, 16, 4),
                                       (5, 300, 520, 516), (2, 300, 1028, 516),
                                       (2, 2049, 4100, 2048), (2, 200, 8196, 260),
                                       (5, 129, 100, 132), (2, 64, 4, 128),
                                       (6, 40, 6160, 2052), (6, 48, 6148, 2048),
                                       (2, 300, 512, 514), (2, 300, 1030, 516),
                                       (2, 130, 1001, 257), (6, 300, 1030, 514),
                                       (6, 200, 3001, 300), (2, 1000, 777, 1001),
                                       (6, 65, 13, 131), (2, 257, 4099, 129)])
def test_dma_kernel_edge_tiles(hip, monkeypatch, cfg, m, k, n):
    monkeypatch.setenv("CLOVE_GEMM_CFG", str(cfg))
    g = rng(cfg * 5 + m + 3 * k + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    bias = g.normal(0, 1, n).astype(np.float32)
    gr = hip.Graph()
    x, wi, bi = gr.input(f"{m},{k}"), gr.input(f"{k},{n}"), gr.input(f"{n}")
    model = gr.compile([gr.op("add", gr.op("matmul", x, wi), bi)])
    ta, tb, tbias = hip.tensor(a), hip.tensor(b), hip.tensor(bias)
    dma = hip.matmul(ta, tb).numpy()
    (dma_fused,) = model.execute([ta, tb, tbias])
    dma_fused = dma_fused.numpy()
    monkeypatch.setenv("CLOVE_GEMM_DMA", "0")
    staged = hip.matmul(ta, tb).numpy()
    (staged_fused,) = model.execute([ta, tb, tbias])
    assert np.array_equal(dma, staged)
    assert np.array_equal(dma_fused, staged_fused.numpy())
    want = oracle.matmul(a, b)
    check(dma, want, f"dma edge cfg {cfg} {m}x{k}x{n}")
    check(dma_fused, oracle.add(want, bias), f"dma edge + bias cfg {cfg} {m}x{k}x{n}")


def test_matmul_random_shapes_sweep(hip):
    """120 seeded random shapes across every plan the GEMM chooses (small,
    strip, skinny, split-K and single-launch tiles in 128x128 and 64x128,
    DMA-staged interior and edge tiles, the 4-byte DMA form for N or K not a
    multiple of 4):
    each product within the matmul bound of the float64 product.  (float64
    stands in for the oracle here to keep the sweep fast; the oracle's own
    f32 result lies within the same bound of it, which the shape tests
    above check.)"""
    g = np.random.default_rng(2024)
    for _ in range(120):
        m = int(g.choice([g.integers(1, 65), g.integers(65, 2500)]))
        k = int(g.choice([g.integers(1, 64), g.integers(64, 2500), 16 * g.integers(4, 160)]))
        n = int(g.choice([g.integers(1, 2500), 4 * g.integers(1, 600), 128 * g.integers(1, 20)]))
        a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
        b = g.normal(0, 1, (k, n)).astype(np.float32)
        got = hip.matmul(hip.tensor(a), hip.tensor(b)).numpy()
        check(got, a.astype(np.float64) @ b.astype(np.float64), f"sweep {m}x{k}x{n}")


@pytest.mark.parametrize("m,k,n", [(300, 512, 516), (32, 4096, 4096)])
@pytest.mark.parametrize("which", ["a", "b"])
def test_tiled_misaligned_operand_falls_back(hip, which, m, k, n):
    """An A or B that is not 16-byte aligned moves one float a lane in the DMA
    kernel's edge form (tiled shapes, 300 x 512 x 516), or takes the
    register-staged kernel where the strip and skinny kernels would read it
    in 8- and 16-byte vectors (32 x 4096 x 4096).  The product is unchanged
    within the matmul bound."""
    g = rng((23 if which == "a" else 24) + m)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    src = a if which == "a" else b
    buf = hip.tensor(np.concatenate([[0.0], src.ravel()]).astype(np.float32))
    view = hip.wrap(buf.device_ptr + 4, src.shape)
    ta = view if which == "a" else hip.tensor(a)
    tb = view if which == "b" else hip.tensor(b)
    check(hip.matmul(ta, tb).numpy(), oracle.matmul(a, b), f"misaligned {which}")
    del view


@pytest.mark.parametrize("m,k,n", [(64, 8192, 4096), (40, 6148, 2048), (64, 4096, 4096),
                                   (48, 8192, 1024), (40, 2048, 40001), (64, 1024, 32000)])
def test_rows_33_to_64_plans(hip, m, k, n):
    """33-64 rows over K > 4096 with N >= 2048, or over N >= 30000, run
    64x128 DMA-staged tiles with the cost model's K split (40 x 2048 x 40001
    on the 4-byte form for its odd N); the others keep the skinny kernel.
    Each within the matmul bound of the oracle, the same bits when
    repeated."""
    g = rng(m + k + n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    check(got, oracle.matmul(a, b), f"plan {m}x{k}x{n}")
    assert np.array_equal(hip.matmul(ta, tb).numpy(), got)


@pytest.mark.parametrize("m,k,n", [
    (3000, 3000, 3000),   # 64x128 tiles, K split two ways; ragged edges and a K tail
    (1536, 1536, 1536),   # 64x128 tiles, four splits
    (2100, 2100, 2100),   # 64x128 tiles, four splits, ragged
    (2048, 2048, 2048),   # 64x128 tiles unsplit (two per CU)
    (256, 4096, 4096),    # 64x128 tiles, six splits
    (16384, 784, 128),    # 64x128 tiles, one per CU over a short K
    (2560, 2560, 2560),   # 128x128 tiles, three splits
    (768, 4096, 4096),    # 64x128 tiles, two splits
    (749, 3725, 1673)])   # K and N odd: 64x128 tiles on the 4-byte DMA form
def test_planner_tile_and_split_choices(hip, m, k, n):
    """Above 64 rows the planner weighs 128x128 against 64x128 tiles and
    the K split by their load balance over the CUs, occupancy and the
    reduce pass.  Sampled row ranges of each resulting plan (first, last,
    and across a 64- and a 128-row tile edge) against the oracle; a
    repeated call gives the same bits."""
    g = rng(m + 5 * k + 11 * n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    for lo, hi in ((0, 3), (62, 66), (126, 130), (m - 3, m)):
        lo, hi = max(0, lo), min(m, hi)
        want = oracle.matmul(a, b, rows=(lo, hi))[lo:hi]
        check(got[lo:hi], want, f"plan {m}x{k}x{n} rows {lo}..{hi}")
    assert np.array_equal(hip.matmul(ta, tb).numpy(), got)


@pytest.mark.parametrize("m,k,n", [
    (1, 4096, 4096),      # skinny kernel, one row in a 32-row block
    (32, 6144, 4096),     # skinny kernel, K past 4096
    (32, 4096, 14336),    # skinny kernel, wide N
    (16, 4096, 50257),    # odd N: skinny with one column block per wave
    (32, 4096, 11008)])   # skinny kernel, N a multiple of 128 but not 4096
def test_decode_shapes_as_planned(hip, m, k, n):
    """Decode-sized products on the paths the plan picks for them, against
    the oracle; a repeated call gives the same bits."""
    g = rng(m + 7 * k + 3 * n)
    a = g.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    b = g.normal(0, 1, (k, n)).astype(np.float32)
    ta, tb = hip.tensor(a), hip.tensor(b)
    got = hip.matmul(ta, tb).numpy()
    check(got, oracle.matmul(a, b), f"decode {m}x{k}x{n}")
    assert np.array_equal(hip.matmul(ta, tb).numpy(), got)


@pytest.mark.parametrize("which", ["a", "b"])
def test_operands_past_2_gib(hip, which):
    """An A or B of 2 GiB or more is past the 32-bit offsets of the buffer
    loads (DMA, strip, skinny), so the product takes the register-staged
    kernel, which indexes in 64 bits.  Rows (A) or columns (B) whose offsets
    lie past 2^31 bytes are checked against the oracle."""
    g = rng(31 if which == "a" else 32)
    if which == "a":
        m, k, n = 140000, 4096, 256
    else:
        m, k, n = 256, 4096, 140000
    a = g.standard_normal((m, k), dtype=np.float32)
    a *= np.float32(1 / 64)
    b = g.standard_normal((k, n), dtype=np.float32)
    got = hip.matmul(hip.tensor(a), hip.tensor(b)).numpy()
    rows = ((0, 2), (131070, 131074), (m - 2, m)) if which == "a" else ((0, 2), (m - 2, m))
    for lo, hi in rows:
        want = oracle.matmul(a, b, rows=(lo, hi))[lo:hi]
        check(got[lo:hi], want, f"{which} past 2 GiB rows {lo}..{hi}")

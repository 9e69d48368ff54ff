"""GPU parity: plans built by the lazy planner (compile/execute).

Config 1 (the 2-layer MLP) runs as one compiled plan and is compared with
the eager CPU composition (Linear::forward, relu, softmax); the tolerance is
the softmax one (1e-4 relative) since the softmax output is what is checked.
"""
import numpy as np
import pytest

import oracle
from clove_amd import workloads
from conftest import assert_close, rng

pytestmark = pytest.mark.gpu


def mlp_graph(hip, batch="64"):
    g = hip.Graph()
    x = g.input(f"{batch},784")
    w1, b1 = g.input("784,128"), g.input("1,128")
    w2, b2 = g.input("128,10"), g.input("1,10")
    h = g.op("relu", g.op("add", g.op("matmul", x, w1), b1))
    y = g.op("softmax", g.op("add", g.op("matmul", h, w2), b2))
    return g, y


def test_config1_mlp_plan(hip):
    x, w1, b1, w2, b2 = workloads.mlp_inputs(0)
    g, y = mlp_graph(hip)
    model = g.compile([y])
    (out,) = model.execute([hip.tensor(v) for v in (x, w1, b1, w2, b2)])
    assert out.shape == (64, 10)
    assert_close(out.numpy(), oracle.mlp_forward(x, w1, b1, w2, b2), 1e-4, 1e-7, "mlp")
    # the same plan again (buffers reused)
    (out2,) = model.execute([hip.tensor(v) for v in (x, w1, b1, w2, b2)])
    assert np.array_equal(out.numpy(), out2.numpy())


def test_symbolic_batch(hip):
    x, w1, b1, w2, b2 = workloads.mlp_inputs(0)
    g, y = mlp_graph(hip, batch="S0")
    model = g.compile([y])
    for bsz in (1, 17, 64):
        (out,) = model.execute([hip.tensor(v) for v in (x[:bsz], w1, b1, w2, b2)], env=[bsz])
        assert_close(out.numpy(), oracle.mlp_forward(x[:bsz], w1, b1, w2, b2), 1e-4, 1e-7,
                     f"batch {bsz}")
    with pytest.raises(hip.CloveError):  # env says 5 rows, input has 17
        model.execute([hip.tensor(v) for v in (x[:17], w1, b1, w2, b2)], env=[5])


def test_chain_with_escaping_values_and_layer_norm(hip):
    gg = rng(3)
    xv = gg.standard_normal((16, 256)).astype(np.float32)
    gam = gg.uniform(0.5, 1.5, 256).astype(np.float32)
    bet = gg.uniform(-0.1, 0.1, 256).astype(np.float32)
    g = hip.Graph()
    x, gm, bt = g.input("16,256"), g.input("256"), g.input("256")
    t = g.op("tanh", x)
    u = g.op("scalar_mul", t, param=2.0)
    ln = g.op("layer_norm", u, gm, bt)
    y = g.op("add", ln, t)
    m = g.compile([y, t])
    out, tt = m.execute([hip.tensor(xv), hip.tensor(gam), hip.tensor(bet)])
    t_ref = oracle.tanh(xv)
    want = oracle.add(oracle.layer_norm(oracle.mul_scalar(t_ref, 2.0), gam, bet), t_ref)
    assert_close(tt.numpy(), t_ref, 1e-5, 1e-6, "escaping tanh")
    assert_close(out.numpy(), want, 1e-4, 1e-5, "chain + layer_norm")


def test_paged_attention_in_graph(hip):
    gg = rng(4)
    B, H, D, bs, nb, mb = 2, 2, 64, 16, 32, 8
    kv = gg.standard_normal((2, nb, bs, H, D)).astype(np.float32)
    q, kn, vn = (gg.standard_normal((B, H * D)).astype(np.float32) for _ in range(3))
    bt = gg.permutation(nb)[: B * mb].reshape(B, mb).astype(np.int32)
    cl = np.array([37, 128], np.int32)
    g = hip.Graph()
    ids = [g.input(f"{B},{H * D}"), g.input(f"{B},{H * D}"), g.input(f"{B},{H * D}"),
           g.input(f"2,{nb},{bs},{H},{D}"), g.input(f"{B},{mb}"), g.input(f"{B}")]
    y = g.op("paged_attention", *ids)
    z = g.op("scalar_mul", y, param=3.0)
    m = g.compile([z])
    (out,) = m.execute([hip.tensor(v) for v in (q, kn, vn, kv, bt, cl)])
    want = oracle.mul_scalar(oracle.paged_attention(q, kn, vn, kv, bt, cl).reshape(B, H * D), 3.0)
    assert_close(out.numpy(), want, 2e-3, 1e-5, "paged in graph")


@pytest.mark.parametrize("m,k,n,bias_n,act", [(64, 784, 128, 128, "relu"), (300, 256, 192, 1, "gelu"),
                                               (130, 96, 10, 3, None), (512, 512, 512, 512, "gelu"),
                                               (16, 1000, 30, 30, "relu")])
def test_gemm_epilogue_fusion(hip, m, k, n, bias_n, act):
    """MatMul -> Add(bias) [-> ReLU/GELU] planned as one GEMM with a fused
    epilogue equals the eager composition: the matmul tolerance on the
    pre-activation, then the elementwise ops applied to the same values."""
    gg = rng(m + n)
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, bias_n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},{k}"), g.input(f"{k},{n}"), g.input(f"{bias_n}")
    y = g.op("add", g.op("matmul", x, wi), bi)
    if act:
        y = g.op(act, y)
    model = g.compile([y])
    assert model.num_steps == 1, model.describe()
    (out,) = model.execute([hip.tensor(v) for v in (a, w, b)])
    pre = oracle.add(oracle.matmul(a, w), b)
    want = getattr(oracle, act)(pre) if act else pre
    atol = 1e-4 * float(np.abs(want).max())
    assert_close(out.numpy(), want, 2e-3, atol, f"fused epilogue {m}x{k}x{n} bias={bias_n} {act}")


@pytest.mark.parametrize("m,k,n,bias_n,act", [(64, 784, 128, 128, "relu"), (32, 4096, 512, 512, "gelu"),
                                               (300, 256, 192, 7, None), (1024, 512, 1024, 1, "gelu"),
                                               (64, 128, 10, 10, None), (70, 100, 50, 1, "relu"),
                                               (40, 1024, 96, 96, "gelu")])
def test_gemm_epilogue_matches_eager_bits(hip, m, k, n, bias_n, act):
    """The fused epilogue rounds in the unfused order: the planned
    GEMM+bias(+act) equals eager matmul, then add, then the activation, bit
    for bit (split-K shapes included: 32x4096 splits K)."""
    gg = rng(7 * m + n)
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, bias_n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},{k}"), g.input(f"{k},{n}"), g.input(f"{bias_n}")
    y = g.op("add", g.op("matmul", x, wi), bi)
    if act:
        y = g.op(act, y)
    model = g.compile([y])
    assert model.num_steps == 1, model.describe()
    ta, tw, tb = hip.tensor(a), hip.tensor(w), hip.tensor(b)
    (fused,) = model.execute([ta, tw, tb])
    eager = hip.add(hip.matmul(ta, tw), tb)
    if act:
        eager = getattr(hip, act)(eager)
    assert np.array_equal(fused.numpy(), eager.numpy())


@pytest.mark.parametrize("cfg", ["5", "4", "2"])  # 128x256, 256x128 and 128x128 tiles
@pytest.mark.parametrize("m,k,n,bias_n,act", [(1000, 64, 1100, 1100, "gelu"),
                                               (1000, 64, 1101, 7, "relu"),
                                               (700, 60, 900, 1, None)])
def test_gemm_epilogue_edge_tiles_large_configs(hip, monkeypatch, cfg, m, k, n, bias_n, act):
    """The fused epilogue on the bounds-checked kernels of the largest tile
    shapes (ragged M and N, K short enough for one split; with N % 4 == 0
    the 128-row tiles take the DMA kernel's edge form): the same bits as
    the eager composition."""
    monkeypatch.setenv("CLOVE_GEMM_CFG", cfg)
    gg = rng(3 * m + n + int(cfg))
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, bias_n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},{k}"), g.input(f"{k},{n}"), g.input(f"{bias_n}")
    y = g.op("add", g.op("matmul", x, wi), bi)
    if act:
        y = g.op(act, y)
    model = g.compile([y])
    assert model.num_steps == 1, model.describe()
    ta, tw, tb = hip.tensor(a), hip.tensor(w), hip.tensor(b)
    (fused,) = model.execute([ta, tw, tb])
    eager = hip.add(hip.matmul(ta, tw), tb)
    if act:
        eager = getattr(hip, act)(eager)
    assert np.array_equal(fused.numpy(), eager.numpy())
    pre = oracle.add(oracle.matmul(a, w), b)
    want = getattr(oracle, act)(pre) if act else pre
    assert_close(fused.numpy(), want, 2e-3, 1e-4 * float(np.abs(want).max()), "edge epilogue")


def test_concurrent_callers(hip):
    """The C ABI serialises host-side calls under one lock; callers on several
    threads get the same results as one caller."""
    import threading

    gg = rng(12)
    xs = [gg.normal(0, 2, (64, 1024)).astype(np.float32) for _ in range(8)]
    want = [oracle.softmax(x) for x in xs]
    got = [None] * 8
    errors = []

    def work(i):
        try:
            for _ in range(5):
                got[i] = hip.softmax(hip.tensor(xs[i])).numpy()
        except Exception as e:  # reported below
            errors.append(e)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t_ in ts:
        t_.start()
    for t_ in ts:
        t_.join()
    assert not errors, errors
    for g_, w in zip(got, want):
        assert_close(g_, w, 1e-4, 1e-9, "threaded softmax")


@pytest.mark.parametrize("plan", ["0,1", "0,3", "1,2"])
@pytest.mark.parametrize("m,k,n,bias_n,act", [(64, 784, 128, 128, "relu"), (32, 4096, 512, 3, "gelu")])
def test_skinny_epilogue(hip, monkeypatch, plan, m, k, n, bias_n, act):
    """The fused epilogue on the skinny path: applied in the kernel (one
    split) or by the split-K reduce, equal to the eager composition's bits."""
    monkeypatch.setenv("CLOVE_GEMM_SKINNY", plan)
    gg = rng(5 * m + n)
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, bias_n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},{k}"), g.input(f"{k},{n}"), g.input(f"{bias_n}")
    y = g.op(act, g.op("add", g.op("matmul", x, wi), bi))
    model = g.compile([y])
    ta, tw, tb = hip.tensor(a), hip.tensor(w), hip.tensor(b)
    (fused,) = model.execute([ta, tw, tb])
    eager = getattr(hip, act)(hip.add(hip.matmul(ta, tw), tb))
    assert np.array_equal(fused.numpy(), eager.numpy())
    want = getattr(oracle, act)(oracle.add(oracle.matmul(a, w), b))
    assert_close(fused.numpy(), want, 2e-3, 1e-4 * float(np.abs(want).max()), "skinny epilogue")


@pytest.mark.parametrize("m,k,n,bias_n,act", [(32, 4096, 512, 3, "gelu"), (20, 300, 66, 66, "relu"),
                                               (32, 4096, 4096, 4096, "relu")])
def test_strip_epilogue(hip, monkeypatch, m, k, n, bias_n, act):
    """The fused epilogue on the strip path (applied at its store), equal to
    the eager composition's bits and to the oracle's composition."""
    monkeypatch.setenv("CLOVE_GEMM_STRIP", "1")
    gg = rng(7 * m + n + k)
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, bias_n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},{k}"), g.input(f"{k},{n}"), g.input(f"{bias_n}")
    y = g.op(act, g.op("add", g.op("matmul", x, wi), bi))
    model = g.compile([y])
    ta, tw, tb = hip.tensor(a), hip.tensor(w), hip.tensor(b)
    (fused,) = model.execute([ta, tw, tb])
    eager = getattr(hip, act)(hip.add(hip.matmul(ta, tw), tb))
    assert np.array_equal(fused.numpy(), eager.numpy())
    want = getattr(oracle, act)(oracle.add(oracle.matmul(a, w), b))
    assert_close(fused.numpy(), want, 2e-3, 1e-4 * float(np.abs(want).max()), "strip epilogue")


@pytest.mark.parametrize("m,k,n,bias_n", [(64, 128, 10, 10), (37, 64, 16, 1), (5, 8, 3, 0),
                                           (64, 128, 17, 17), (64, 2048, 10, 10),
                                           (300, 96, 12, 12)])
def test_gemm_softmax_head(hip, m, k, n, bias_n):
    """MatMul [-> Add] -> Softmax planned as one step.  N <= 16 on the small
    GEMM path applies the row softmax in the GEMM's epilogue; N = 17 and
    K = 2048 (tiled path) run the product then the row kernel.  The softmax
    tolerance, against the oracle's composition."""
    gg = rng(3 * m + k + n)
    a = gg.normal(0, 1 / np.sqrt(k), (m, k)).astype(np.float32)
    w = gg.normal(0, 1, (k, n)).astype(np.float32)
    b = gg.normal(0, 1, max(bias_n, 1)).astype(np.float32)
    g = hip.Graph()
    x, wi = g.input(f"{m},{k}"), g.input(f"{k},{n}")
    y = g.op("matmul", x, wi)
    ins = [a, w]
    if bias_n:
        bi = g.input(f"{bias_n}")
        y = g.op("add", y, bi)
        ins.append(b)
    model = g.compile([g.op("softmax", y)])
    assert model.num_steps == 1, model.describe()
    (out,) = model.execute([hip.tensor(v) for v in ins])
    pre = oracle.matmul(a, w)
    if bias_n:
        pre = oracle.add(pre, b)
    assert_close(out.numpy(), oracle.softmax(pre), 1e-4, 1e-7, f"softmax head {m}x{k}x{n}")


@pytest.mark.parametrize("act", [None, "relu", "gelu", "softmax"])
def test_gemm_k0_epilogue(hip, act):
    """K = 0: the product is zero and the fused epilogue still applies
    (act(0 + bias), or the row softmax of the bias)."""
    m, n = 5, 7
    b = rng(93).normal(0, 1, n).astype(np.float32)
    g = hip.Graph()
    x, wi, bi = g.input(f"{m},0"), g.input(f"0,{n}"), g.input(f"{n}")
    y = g.op("add", g.op("matmul", x, wi), bi)
    if act:
        y = g.op(act, y)
    model = g.compile([y])
    assert model.num_steps == 1, model.describe()
    (out,) = model.execute([hip.tensor(np.zeros((m, 0), np.float32)),
                            hip.tensor(np.zeros((0, n), np.float32)), hip.tensor(b)])
    pre = np.broadcast_to(b, (m, n)).astype(np.float32)
    want = getattr(oracle, act)(pre) if act else pre
    assert_close(out.numpy(), want, 1e-5, 1e-7, f"K=0 {act}")
    z = hip.matmul(hip.tensor(np.zeros((m, 0), np.float32)),
                   hip.tensor(np.zeros((0, n), np.float32))).numpy()
    assert z.shape == (m, n) and np.all(z == 0)


def test_horizontal_matmul_group(hip):
    """Independent MatMuls (lazy.rs:2443-2493) run as one grouped launch:
    a Q/K/V-style projection of one input with bias, ReLU and a softmax
    head, plus a K = 2048 product that the group runs on its own.  Each
    output matches the eager composition bit for bit (the same per-wave K
    ranges as a single launch) and the oracle within the matmul bound."""
    S, E = 37, 64
    gg = rng(94)
    x = gg.normal(0, 1 / 8, (S, E)).astype(np.float32)
    y = gg.normal(0, 1 / 45, (S, 2048)).astype(np.float32)
    wq, wk = (gg.normal(0, 1, (E, E)).astype(np.float32) for _ in range(2))
    wv = gg.normal(0, 1, (E, 32)).astype(np.float32)
    wh = gg.normal(0, 1, (E, 10)).astype(np.float32)
    wy = gg.normal(0, 1, (2048, 16)).astype(np.float32)
    bq = gg.normal(0, 1, E).astype(np.float32)
    bh = gg.normal(0, 1, 10).astype(np.float32)
    g = hip.Graph()
    ix, iy = g.input(f"{S},{E}"), g.input(f"{S},2048")
    iwq, iwk, iwv, iwh, iwy = (g.input(f"{a},{b}") for a, b in
                               ((E, E), (E, E), (E, 32), (E, 10), (2048, 16)))
    ibq, ibh = g.input(f"{E}"), g.input("10")
    q = g.op("add", g.op("matmul", ix, iwq), ibq)
    k = g.op("relu", g.op("matmul", ix, iwk))
    v = g.op("matmul", ix, iwv)
    h = g.op("softmax", g.op("add", g.op("matmul", ix, iwh), ibh))
    z = g.op("matmul", iy, iwy)
    model = g.compile([q, k, v, h, z])
    assert model.num_steps == 1 and model.describe().startswith("MatMulGroup["), model.describe()
    t = hip.tensor
    ins = [t(a) for a in (x, y, wq, wk, wv, wh, wy, bq, bh)]
    outs = [o.numpy() for o in model.execute(ins)]
    tx, ty, twq, twk, twv, twh, twy, tbq, tbh = ins
    eager = [hip.add(hip.matmul(tx, twq), tbq), hip.relu(hip.matmul(tx, twk)),
             hip.matmul(tx, twv), None, hip.matmul(ty, twy)]
    for i, e in enumerate(eager):
        if e is not None:
            assert np.array_equal(outs[i], e.numpy()), f"member {i} differs from eager"
    want = [oracle.add(oracle.matmul(x, wq), bq), oracle.relu(oracle.matmul(x, wk)),
            oracle.matmul(x, wv), oracle.softmax(oracle.add(oracle.matmul(x, wh), bh)),
            oracle.matmul(y, wy)]
    for i, (got, w_) in enumerate(zip(outs, want)):
        if i == 3:
            assert_close(got, w_, 1e-4, 1e-7, "softmax head member")
        else:
            assert_close(got, w_, 2e-3, 1e-4 * float(np.abs(w_).max()), f"member {i}")


# ---------------------------------------------------------------------------
# chains past one launch's limits (16 inputs, 16 stored values)
# ---------------------------------------------------------------------------

def test_sum_of_twenty_inputs(hip):
    g = hip.Graph()
    xs = rng(40).standard_normal((20, 64, 96)).astype(np.float32)
    ids = [g.input("64,96") for _ in range(20)]
    acc = ids[0]
    for i in ids[1:]:
        acc = g.op("add", acc, i)
    m = g.compile([acc])
    assert m.num_steps == 2
    (got,) = m.execute([hip.tensor(x) for x in xs])
    want = xs[0]
    for x in xs[1:]:
        want = oracle.add(want, x)      # the same sequential f32 order
    assert np.array_equal(got.numpy(), want)


def test_twenty_requested_values_of_one_chain(hip):
    g = hip.Graph()
    x = rng(41).standard_normal((33, 17)).astype(np.float32)
    xi = g.input("33,17")
    ids, v = [], xi
    for i in range(20):
        v = g.op("sin" if i % 2 else "cos", v)
        ids.append(v)
    m = g.compile(ids)
    outs = m.execute([hip.tensor(x)])
    want = x
    for i, o in enumerate(outs):
        want = oracle.sin(want) if i % 2 else oracle.cos(want)
        assert_close(o.numpy(), want, 1e-5, 1e-6, f"value {i}")


# ---------------------------------------------------------------------------
# the FlashAttention pattern (lazy.rs:1621-1690) as one planned step
# ---------------------------------------------------------------------------

def attention_plan(hip, S, Sk, X, D, q_pos, k_pos, scale):
    g = hip.Graph()
    q, k, v = g.input(f"{S},{X}"), g.input(f"{Sk},{X}"), g.input(f"{Sk},{X}")
    qr, kr = g.rope(q, D, q_pos), g.rope(k, D, k_pos)
    qs = g.op("scalar_mul", qr, param=scale) if scale else qr
    y = g.op("matmul", g.op("softmax", g.op("matmul", qs, kr)), v)
    m = g.compile([y])
    assert m.num_steps == 1 and m.describe().startswith("FlashAttention"), m.describe()
    return m


def attention_want(q, k, v, D, q_pos, k_pos, scale, rows=None):
    """The reference kernel's contract (lazy.rs:4821-4909): q and k rotated
    at their RoPE positions, keys after the query's row masked."""
    qr, kr = oracle.rope(q, D, q_pos), oracle.rope(k, D, k_pos)
    return oracle.attention(qr, kr, v, q.shape[-1] // D, 0, 0, oracle.ATTN_CAUSAL,
                            scale or None, rows=rows)


@pytest.mark.parametrize("S,Sk,X,D,q_pos,k_pos,scale", [
    (64, 64, 64, 64, 0, 0, 0.125),        # one head, MultiHeadAttention's scale
    (130, 130, 256, 128, 3, 3, None),     # two heads, no ScalarMul: 1/sqrt(D)
    (100, 100, 192, 64, 5, 17, 0.2),      # different rotation positions, own scale
    (33, 70, 128, 64, 0, 9, 1.0),         # more keys than queries
])
def test_graph_flash_attention(hip, S, Sk, X, D, q_pos, k_pos, scale):
    g = rng(S * 3 + Sk + X + D)
    q = g.standard_normal((S, X)).astype(np.float32)
    k = g.standard_normal((Sk, X)).astype(np.float32)
    v = g.standard_normal((Sk, X)).astype(np.float32)
    m = attention_plan(hip, S, Sk, X, D, q_pos, k_pos, scale)
    (got,) = m.execute([hip.tensor(a) for a in (q, k, v)])
    want = attention_want(q, k, v, D, q_pos, k_pos, scale)
    assert_close(got.numpy(), want, 2e-3, 1e-5, f"attention plan S={S} Sk={Sk} X={X} D={D}")


def test_graph_flash_attention_equals_eager_bits(hip):
    """With equal positions the index mask is the position mask, so the
    planned step and the eager entry give the same bits."""
    g = rng(77)
    q, k, v = (g.standard_normal((257, 256)).astype(np.float32) for _ in range(3))
    m = attention_plan(hip, 257, 257, 256, 128, 11, 11, None)
    t = hip.tensor
    (got,) = m.execute([t(q), t(k), t(v)])
    eager = hip.flash_attention(t(q), t(k), t(v), 2, 11, 11, hip.ATTN_CAUSAL | hip.ATTN_ROPE)
    assert np.array_equal(got.numpy(), eager.numpy())


def test_graph_flash_attention_4096_sampled(hip):
    """S = 4096, hidden 4096 = 32 heads of 128: sampled query rows of every
    head against the oracle."""
    g = rng(78)
    S, X, D = 4096, 4096, 128
    q, k, v = (g.standard_normal((S, X)).astype(np.float32) for _ in range(3))
    m = attention_plan(hip, S, S, X, D, 0, 0, float(1 / np.sqrt(np.float32(D))))
    (got,) = m.execute([hip.tensor(a) for a in (q, k, v)])
    got = got.numpy()
    for lo, hi in ((0, 2), (127, 130), (2047, 2049), (4094, 4096)):
        want = attention_want(q, k, v, D, 0, 0, float(1 / np.sqrt(np.float32(D))),
                              rows=(lo, hi))
        assert_close(got[lo:hi], want[lo:hi], 2e-3, 1e-5, f"rows {lo}..{hi}")


def test_graph_attention_non_match_runs_op_by_op(hip):
    """Without RoPE on k the nodes run one by one with the matmul rule (k is
    [D, Sk], the keys transposed), the graph's literal meaning."""
    g = rng(79)
    q = g.standard_normal((64, 128)).astype(np.float32)
    kt = g.standard_normal((128, 64)).astype(np.float32)
    v = g.standard_normal((64, 128)).astype(np.float32)
    gr = hip.Graph()
    qi, ki, vi = gr.input("64,128"), gr.input("128,64"), gr.input("64,128")
    y = gr.op("matmul", gr.op("softmax", gr.op("matmul", gr.rope(qi, 64, 2), ki)), vi)
    m = gr.compile([y])
    assert "FlashAttention" not in m.describe()
    (got,) = m.execute([hip.tensor(a) for a in (q, kt, v)])
    scores = oracle.softmax(oracle.matmul(oracle.rope(q, 64, 2), kt))
    want = oracle.matmul(scores, v)
    assert_close(got.numpy(), want, 2e-3, 1e-4 * float(np.abs(want).max()), "op by op")

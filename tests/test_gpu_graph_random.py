"""GPU parity: seeded random elementwise graphs through the planner.

Each case draws a DAG of unary ops (relu, gelu, sigmoid, tanh, sin, cos,
scalar_mul), binary ops with broadcast operands (b read as b[i % numel(b)],
backend.rs:1483-1493), softmax and layer norm, over a random (R, C) shape
and inputs of four broadcast classes: full, (C,), (1, C) and a flat length
that need not divide R*C.  A random subset of the values is requested, so
intermediates escape fused chains and chains split at the reductions.  The
compiled plan's outputs are compared with the oracle evaluated op by op in
f32, as the eager CPU path computes them (2e-5 relative plus 2e-5 of the
output's largest magnitude: the chains are short and stay within |x| <= 2,
so the GPU's fused f32 and its own transcendentals stay within a few ulps).
"""
import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu

UNARY = ["relu", "gelu", "sigmoid", "tanh", "sin", "cos", "scalar_mul"]
BINARY = ["add", "sub", "mul"]


def random_graph(seed):
    """Returns (input shapes, input values, nodes, oracle values, outputs);
    a node is ("in", index, None) or (op, dependency indices, param)."""
    g = rng(seed)
    R, C = int(g.integers(1, 300)), int(g.integers(1, 700))
    shapes = []
    for i in range(int(g.integers(1, 7))):
        kind = g.integers(0, 4) if i else 0
        shapes.append((int(g.integers(1, R * C + 1)),) if kind == 3 else [(R, C), (C,), (1, C)][kind])
    n_in = len(shapes)
    vals = [g.uniform(-2, 2, s).astype(np.float32) for s in shapes]
    nodes = [("in", i, None) for i in range(n_in)]
    ref = list(vals)
    for _ in range(int(g.integers(1, 14))):
        r = g.random()
        full = [i for i, v in enumerate(ref) if v.shape == (R, C)]
        if r < 0.08 and full:
            x = int(g.choice(full))
            nodes.append(("softmax", (x,), None))
            ref.append(oracle.softmax(ref[x]))
        elif r < 0.14 and full:
            x = int(g.choice(full))
            gamma = g.uniform(0.5, 1.5, C).astype(np.float32)
            beta = g.uniform(-0.2, 0.2, C).astype(np.float32)
            gi = len(ref)
            for v in (gamma, beta):
                nodes.append(("in", len(shapes), None))
                shapes.append((C,))
                vals.append(v)
                ref.append(v)
            nodes.append(("layer_norm", (x, gi, gi + 1), None))
            ref.append(oracle.layer_norm(ref[x], gamma, beta))
        elif r < 0.55:
            name = str(g.choice(UNARY))
            x = int(g.integers(0, len(ref)))
            if name == "scalar_mul":
                p = float(np.float32(g.uniform(-1.5, 1.5)))
                nodes.append((name, (x,), p))
                ref.append(oracle.mul_scalar(ref[x], p))
            else:
                nodes.append((name, (x,), None))
                ref.append(getattr(oracle, name)(ref[x]))
        else:
            name = str(g.choice(BINARY))
            a = int(g.choice(full)) if full and g.random() < 0.8 else int(g.integers(0, len(ref)))
            b = int(g.integers(0, len(ref)))
            nodes.append((name, (a, b), None))
            ref.append(getattr(oracle, name)(ref[a], ref[b]))
    n = len(nodes)
    pool = np.arange(n_in, n) if n > n_in else np.arange(n)
    outs = sorted(set(int(x) for x in g.choice(pool, int(g.integers(1, min(6, n) + 1)))))
    if n - 1 not in outs:
        outs.append(n - 1)
    return shapes, vals, nodes, ref, outs


@pytest.mark.parametrize("seed", range(40))
def test_random_graph(hip, seed):
    shapes, vals, nodes, ref, outs = random_graph(1000 + seed)
    gr = hip.Graph()
    ids = []
    for kind, deps, p in nodes:
        if kind == "in":
            ids.append(gr.input(shapes[deps]))
        elif kind == "scalar_mul":
            ids.append(gr.op(kind, ids[deps[0]], param=p))
        else:
            ids.append(gr.op(kind, *[ids[d] for d in deps]))
    m = gr.compile([ids[o] for o in outs])
    got = m.execute([hip.tensor(v) for v in vals])
    for o, t in zip(outs, got):
        want = ref[o].astype(np.float64)
        assert t.shape == want.shape, (o, t.shape, want.shape)
        have = t.numpy().astype(np.float64)
        tol = 2e-5 * np.abs(want) + 2e-5 * max(1.0, float(np.abs(want).max()))
        err = np.abs(have - want)
        i = int(np.argmax(err - tol))
        assert np.all(err <= tol), (
            f"node {o} ({nodes[o][0]}): {have.ravel()[i]} vs {want.ravel()[i]}; "
            f"plan {m.describe()}")

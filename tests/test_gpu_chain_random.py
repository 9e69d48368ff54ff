"""GPU parity: seeded random fused chains against the oracle's op-by-op
evaluation (one materialised f32 pass per op, as Clove's eager CPU path).

Each case draws an output length (odd, multiple of 4, or past a 64 Ki
boundary), one to five inputs, each full length or a shorter one read as
x[i % len] (any length, not only divisors), and a chain of 1-8 ops from
add/sub/mul, scalar_mul and the unary ops, some of whose intermediate
values are stored as extra outputs.  A binary op's first operand is always
full length (an earlier value or a full input), as in the chains the planner
builds.  Arithmetic is bit-exact on both sides; each transcendental op
(gelu, sigmoid, tanh, sin, cos) may differ by a few ulp, so the bound grows
with their number in the chain: |g - c| <= k (1e-6 max(1, |c|max) + 1e-5 |c|)
with k = 1 + transcendental ops.
"""
import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu

UNARY = ["relu", "gelu", "sigmoid", "tanh", "sin", "cos"]
BINARY = ["add", "sub", "mul"]


def random_chain(seed):
    g = rng(seed)
    n = int(g.choice([g.integers(1, 64), 4 * g.integers(1, 20000), g.integers(65536, 70000)]))
    k = int(g.integers(1, 6))
    sizes = [n] + [n if g.random() < 0.5 else int(g.integers(1, n + 1)) for _ in range(k - 1)]
    inputs = [g.standard_normal(s).astype(np.float32) for s in sizes]
    full = [-(i + 1) for i, s in enumerate(sizes) if s == n]
    ops = []
    trans = 0
    for i in range(int(g.integers(1, 9))):
        # a full-length operand: an earlier value or a full input
        s0 = int(g.integers(0, i)) if i and g.random() < 0.7 else int(g.choice(full))
        store = bool(g.random() < 0.3)
        r = g.random()
        if r < 0.45:
            s1 = int(g.integers(0, i)) if i and g.random() < 0.3 else -int(g.integers(1, k + 1))
            ops.append((str(g.choice(BINARY)), s0, s1, store))
        elif r < 0.6:
            ops.append(("scalar_mul", s0, 0, store, float(np.float32(g.uniform(-2, 2)))))
        else:
            name = str(g.choice(UNARY))
            trans += name != "relu"
            ops.append((name, s0, 0, store))
    # pass only the inputs the chain reads, renumbered in order of index
    def refs(op):
        return [op[1]] + ([op[2]] if op[0] in BINARY else [])
    used = sorted({-r for op in ops for r in refs(op) if r < 0})
    new_ref = {-old: -(j + 1) for j, old in enumerate(used)}
    ops = [(op[0], new_ref.get(op[1], op[1]),
            new_ref.get(op[2], op[2]) if op[0] in BINARY else op[2]) + tuple(op[3:])
           for op in ops]
    return n, [inputs[i - 1] for i in used], ops, trans


@pytest.mark.parametrize("seed", range(32))
def test_random_chain(hip, seed):
    n, inputs, ops, trans = random_chain(2000 + seed)
    got = hip.fused_chain(ops, [hip.tensor(x) for x in inputs])
    want = oracle.chain(ops, inputs)
    assert len(got) == len(want), f"seed {seed}: {len(got)} outputs, want {len(want)}"
    k = 1 + trans
    for j, (g_, w) in enumerate(zip(got, want)):
        g_ = g_.numpy().astype(np.float64)
        w = np.asarray(w, np.float64)
        assert g_.shape == w.shape, f"seed {seed} output {j}: shape {g_.shape} != {w.shape}"
        bound = k * (1e-6 * max(1.0, float(np.abs(w).max(initial=0.0))) + 1e-5 * np.abs(w))
        err = np.abs(g_ - w)
        assert np.all(err <= bound), (
            f"seed {seed} output {j}: n={n} sizes={[x.size for x in inputs]} ops={ops}: "
            f"max excess {np.max(err - bound):.3e}")

"""GPU parity: the fused AdamW update vs the oracle (optim.rs:375-395).

The kernel follows the CPU branch's operand order with IEEE division and
square root and the host's powf for the bias corrections, so it is checked
bit for bit over several steps."""
import numpy as np
import pytest

import oracle
from conftest import rng

pytestmark = pytest.mark.gpu


def run_steps(hip, sizes, steps, seed, **hyper):
    g = rng(seed)
    ws = [g.standard_normal(n).astype(np.float32) for n in sizes]
    tw = [hip.tensor(w) if w.size else hip.empty((0,)) for w in ws]
    tm = [hip.tensor(np.zeros(w.size, np.float32)) if w.size else hip.empty((0,)) for w in ws]
    tv = [hip.tensor(np.zeros(w.size, np.float32)) if w.size else hip.empty((0,)) for w in ws]
    ms = [np.zeros_like(w) for w in ws]
    vs = [np.zeros_like(w) for w in ws]
    for t in range(1, steps + 1):
        grads = [(g.standard_normal(w.size) * 65536 * 0.8).astype(np.float32) for w in ws]
        tg = [hip.tensor(x) if x.size else hip.empty((0,)) for x in grads]
        hip.adamw_step(tw, tg, tm, tv, t, **hyper)
        for i in range(len(ws)):
            ws[i], ms[i], vs[i] = oracle.adamw(ws[i], grads[i], ms[i], vs[i], t, **hyper)
    return tw, tm, tv, ws, ms, vs


@pytest.mark.parametrize("sizes", [[1], [3, 5, 4099], [1 << 20], [0, 7],
                                   [i * 13 + 1 for i in range(20)]])
def test_adamw_bit_exact(hip, sizes):
    tw, tm, tv, ws, ms, vs = run_steps(hip, sizes, 4, sum(sizes) + 1)
    for i in range(len(sizes)):
        if sizes[i] == 0:
            continue
        assert np.array_equal(tw[i].numpy(), ws[i]), f"w[{i}]"
        assert np.array_equal(tm[i].numpy(), ms[i]), f"m[{i}]"
        assert np.array_equal(tv[i].numpy(), vs[i]), f"v[{i}]"


def test_adamw_hyperparameters_and_misaligned(hip):
    g = rng(70)
    n = 1001
    w = g.standard_normal(n).astype(np.float32)
    gr = (g.standard_normal(n) * 3).astype(np.float32)
    # a borrowed view 4 bytes into a buffer: not 16-byte aligned (scalar path)
    buf = hip.tensor(np.concatenate([[0.0], w]).astype(np.float32))
    tw = hip.wrap(buf.device_ptr + 4, (n,))
    tm, tv = hip.tensor(np.zeros(n, np.float32)), hip.tensor(np.zeros(n, np.float32))
    hyper = dict(lr=0.05, beta1=0.8, beta2=0.99, eps=1e-6, weight_decay=0.1, loss_scale=2.0,
                 clip=0.5)
    hip.adamw_step([tw], [hip.tensor(gr)], [tm], [tv], 3, **hyper)
    we, me, ve = oracle.adamw(w, gr, np.zeros(n, np.float32), np.zeros(n, np.float32), 3, **hyper)
    assert np.array_equal(tw.numpy(), we)
    assert np.array_equal(tm.numpy(), me) and np.array_equal(tv.numpy(), ve)
    del tw


def test_adamw_errors(hip):
    a, b = hip.tensor(np.ones(4, np.float32)), hip.tensor(np.ones(5, np.float32))
    with pytest.raises(hip.CloveError):
        hip.adamw_step([a], [b], [a], [a], 1)
    with pytest.raises(hip.CloveError):
        hip.adamw_step([a], [a], [a], [a], 0)


@pytest.mark.parametrize("seed", range(8))
def test_adamw_random_bit_exact(hip, seed):
    """Seeded launches of 1-16 parameter tensors of random sizes (the most
    one launch carries), random hyperparameters and gradient scales, three
    steps each, bit for bit against the oracle."""
    g = rng(4000 + seed)
    sizes = [int(g.choice([g.integers(1, 64), g.integers(64, 5000), g.integers(5000, 300000)]))
             for _ in range(int(g.integers(1, 17)))]
    hyper = dict(lr=float(np.float32(g.uniform(1e-4, 0.1))),
                 beta1=float(np.float32(g.uniform(0.8, 0.95))),
                 beta2=float(np.float32(g.uniform(0.9, 0.9999))),
                 eps=float(np.float32(10 ** g.uniform(-9, -5))),
                 weight_decay=float(np.float32(g.uniform(0, 0.1))),
                 loss_scale=float(np.float32(2 ** int(g.integers(0, 17)))),
                 clip=float(np.float32(g.uniform(0.1, 2.0))))
    tw, tm, tv, ws, ms, vs = run_steps(hip, sizes, 3, 4100 + seed, **hyper)
    for i in range(len(sizes)):
        assert np.array_equal(tw[i].numpy(), ws[i]), f"seed {seed} w[{i}] ({sizes[i]}) {hyper}"
        assert np.array_equal(tm[i].numpy(), ms[i]), f"seed {seed} m[{i}]"
        assert np.array_equal(tv[i].numpy(), vs[i]), f"seed {seed} v[{i}]"

"""The C-ABI boundary on the CPU: the library loads, exports every symbol the
header declares, reports errors as status codes instead of aborting, and the
lazy planner builds the expected plans (planning touches no device)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import clove_amd as ca
from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "clove_hip.h")


@pytest.fixture(scope="module", autouse=True)
def built_library():
    if not os.path.exists(ca.LIB_PATH):
        import __graft_entry__

        __graft_entry__.build()
    return ca.lib()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(clove_hip_\w+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for required in ("clove_hip_init", "clove_hip_tensor_create", "clove_hip_tensor_data",
                     "clove_hip_tensor_free", "clove_hip_add", "clove_hip_sub", "clove_hip_mul",
                     "clove_hip_mul_scalar", "clove_hip_relu", "clove_hip_gelu",
                     "clove_hip_sigmoid", "clove_hip_tanh", "clove_hip_sin", "clove_hip_cos",
                     "clove_hip_softmax", "clove_hip_layer_norm", "clove_hip_matmul",
                     "clove_hip_paged_attention", "clove_hip_paged_gather_indices",
                     "clove_hip_fused_chain", "clove_hip_compile", "clove_hip_execute"):
        assert required in names


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", ca.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\sT\s(clove_hip_\w+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # ...and the Python binding declares a signature for each of them.
    lib = ca.lib()
    for n in declared_functions():
        assert getattr(lib, n).argtypes is not None, n


def test_calls_before_init_fail_with_status():
    lib = ca.lib()
    shape = (C.c_size_t * 2)(2, 3)
    p = lib.clove_hip_tensor_empty(shape, 2, ca.F32)
    assert not p
    assert lib.clove_hip_last_status() == ca.ERR_NOT_INIT
    assert "clove_hip_init" in ca.last_error()
    assert lib.clove_hip_synchronize() == ca.ERR_NOT_INIT


def test_null_handles_are_errors_not_crashes():
    lib = ca.lib()
    assert not lib.clove_hip_add(None, None)
    assert lib.clove_hip_last_status() == ca.ERR_INVALID
    assert not lib.clove_hip_tensor_create(None, 2, 2)        # ffi.rs:78-80
    assert lib.clove_hip_tensor_data(None, None) == ca.ERR_INVALID
    lib.clove_hip_tensor_free(None)                           # ffi.rs:91-96: ignored
    assert not lib.clove_hip_paged_attention(None, None, None, None, None, None)


# ---------------------------------------------------------------------------
# planner (lazy.rs:1553-2535), CPU only
# ---------------------------------------------------------------------------

def steps(model):
    return [line.split(" ")[0] for line in model.describe().strip().splitlines()[:-1]]


def mlp_graph():
    g = ca.Graph()
    x = g.input("S0,784")
    w1 = g.input("784,128")
    b1 = g.input("1,128")
    w2 = g.input("128,10")
    b2 = g.input("1,10")
    h = g.op("relu", g.op("add", g.op("matmul", x, w1), b1))
    y = g.op("softmax", g.op("add", g.op("matmul", h, w2), b2))
    return g, y


def test_plan_mlp():
    # Linear::forward (matmul then bias add, nn.rs:115-118) and the ReLU fold
    # into the GEMM's epilogue; the classifier head's softmax folds into the
    # second GEMM (a row softmax over the last dim).
    g, y = mlp_graph()
    m = g.compile([y])
    assert steps(m) == ["MatMul+Add+ReLU", "MatMul+Add+Softmax"]
    assert m.num_steps == 2
    # liveness: the hidden layer's buffer is reused once the second GEMM has
    # read it
    assert "vbufs=2" in m.describe()


def test_plan_epilogue_fusion_only_for_sole_consumers():
    g = ca.Graph()
    x, w, b = g.input("4,8"), g.input("8,6"), g.input("6")
    mm = g.op("matmul", x, w)
    add = g.op("add", mm, b)
    act = g.op("gelu", add)
    both = g.op("mul", act, add)     # add has a second consumer: GELU stays unfused
    m = g.compile([both])
    assert steps(m) == ["MatMul+Add", "Fused[GELU,Mul]"]
    g2 = ca.Graph()
    x, w, b = g2.input("4,8"), g2.input("8,6"), g2.input("6")
    mm = g2.op("matmul", x, w)
    y = g2.op("add", b, mm)          # bias first: shape follows b, no fusion
    m2 = g2.compile([y, mm])
    assert steps(m2) == ["MatMul", "Fused[Add]"]


def test_plan_horizontal_matmul_group():
    # lazy.rs:2443-2493: consecutive MatMul steps none of which reads another's
    # output form one group (here a Q/K/V projection of one input, each with
    # its own epilogue); a MatMul reading a member's output ends the group.
    g = ca.Graph()
    x = g.input("S0,64")
    wq, wk, wv, bq = g.input("64,64"), g.input("64,64"), g.input("64,32"), g.input("64")
    q = g.op("add", g.op("matmul", x, wq), bq)
    k = g.op("relu", g.op("matmul", x, wk))
    v = g.op("matmul", x, wv)
    z = g.op("matmul", q, wk)                       # reads q: not in the group
    m = g.compile([q, k, v, z])
    assert steps(m) == ["MatMulGroup[MatMul+Add,MatMul+ReLU,MatMul]", "MatMul"]
    # the shared input x is listed once among the group's inputs
    first = m.describe().splitlines()[0]
    ins = first[first.index("in=(") + 4:first.index(")")].split(",")
    assert len(ins) == len(set(ins)) == 5


def test_plan_dependent_matmuls_stay_apart():
    g = ca.Graph()
    x, w1, w2, w3 = g.input("4,8"), g.input("8,8"), g.input("8,8"), g.input("8,8")
    a = g.op("matmul", x, w1)
    b = g.op("matmul", x, w2)
    c = g.op("matmul", b, w3)                       # reads the second member
    m = g.compile([a, c])
    assert steps(m) == ["MatMulGroup[MatMul,MatMul]", "MatMul"]


def test_plan_dce_and_constant_folding():
    g = ca.Graph()
    a = g.input("4,4")
    b = g.input("4,4")
    dead = g.op("gelu", g.op("sin", a))             # not an output: removed
    s = g.op("scalar_mul", a, param=1.0)            # x * 1.0: folded away
    y = g.op("mul", g.op("add", s, b), b)
    m = g.compile([y])
    d = m.describe()
    assert steps(m) == ["Fused[Add,Mul]"]
    assert "folded=1" in d
    assert "Sin" not in d and "GELU" not in d and "ScalarMul" not in d
    del dead


def test_plan_barriers_and_escaping_values():
    g = ca.Graph()
    x = g.input("8,16")
    gam = g.input("16")
    bet = g.input("16")
    t = g.op("tanh", x)
    u = g.op("mul_scalar" if False else "scalar_mul", t, param=2.0)
    ln = g.op("layer_norm", u, gam, bet)
    y = g.op("add", ln, t)            # t escapes the first chain
    m = g.compile([y])
    lines = m.describe().strip().splitlines()
    assert steps(m) == ["Fused[Tanh,ScalarMul]", "LayerNorm", "Fused[Add]"]
    assert re.search(rf"out=\({t},{u}\)", lines[0]), lines[0]


def test_plan_splits_chains_on_shape_change():
    g = ca.Graph()
    a = g.input("4,8")
    f = g.op("flatten", a)            # [1, 32]: same numel, joins the chain
    b = g.input("3")
    c = g.op("add", b, b)             # 3 elements: a new chain
    m = g.compile([f, c])
    assert steps(m) == ["Fused[Flatten]", "Fused[Add]"]


def test_symbolic_shapes_parse_and_reject():
    g = ca.Graph()
    g.input("S0*16+2,(S1-1)*4")
    for bad in ("", "S4", "3,,4", "2*", "x"):
        with pytest.raises(ca.CloveError):
            g.input(bad)
    with pytest.raises(ca.CloveError):
        g.op("matmul", 0)             # wrong operand count
    with pytest.raises(ca.CloveError):
        g.op("add", 0, 99)            # unknown node

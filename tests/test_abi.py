"""The C-ABI boundary on the CPU: the library loads, exports every symbol the
header declares, reports errors as status codes instead of aborting, and the
lazy planner builds the expected plans (planning touches no device)."""
import ctypes as C
import os
import re
import subprocess
import sys

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


def header_arities():
    """Parameter count of every function the header declares."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for name, params in re.findall(r"\b(clove_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_integration_rust_block_matches_the_header():
    """The Rust `extern "C"` block a maintainer copies declares every entry
    of the header, with the same number of parameters."""
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = doc[doc.index('extern "C" {'):]
    block = block[:block.index("\n}")]
    rust = {}
    for name, params in re.findall(r"pub fn (clove_hip_\w+)\(([^)]*)\)", block, flags=re.S):
        params = re.sub(r"//[^\n]*", "", params).strip().rstrip(",")
        rust[name] = 0 if not params else params.count(",") + 1
    header = header_arities()
    assert header and set(header) == set(declared_functions())
    assert sorted(set(header) - set(rust)) == [], "missing from the Rust extern block"
    assert sorted(set(rust) - set(header)) == [], "not in the header"
    wrong = {n: (header[n], rust[n]) for n in header if header[n] != rust[n]}
    assert not wrong, f"parameter counts differ (header, rust): {wrong}"


def test_calls_before_init_fail_with_status():
    """In a fresh process (in this one a GPU test may already have called
    clove_hip_init): calls before init fail with ERR_NOT_INIT."""
    code = (
        "import sys, ctypes as C; sys.path.insert(0, %r)\n"
        "import clove_amd as ca\n"
        "lib = ca.lib()\n"
        "shape = (C.c_size_t * 2)(2, 3)\n"
        "assert not lib.clove_hip_tensor_empty(shape, 2, ca.F32)\n"
        "assert lib.clove_hip_last_status() == ca.ERR_NOT_INIT\n"
        "assert 'clove_hip_init' in ca.last_error()\n"
        "assert lib.clove_hip_synchronize() == ca.ERR_NOT_INIT\n"
        "print('ok')\n" % ROOT)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.strip() == "ok", (r.stdout, r.stderr[-2000:])


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


# ---------------------------------------------------------------------------
# fused-chain structure checks (before any operand is followed), CPU only
# ---------------------------------------------------------------------------

def _chain_status(ops, n_inputs=1):
    lib = ca.lib()
    arr = (ca.ChainOp * len(ops))()
    for i, (name, s0, s1) in enumerate(ops):
        arr[i] = ca.ChainOp(ca.OP[name.upper()], s0, s1, 0, 0.0)
    ins = (C.c_void_p * n_inputs)()          # NULL handles: structure is checked first
    outs = (C.c_void_p * len(ops))()
    return lib.clove_hip_fused_chain(arr, len(ops), ins, n_inputs, outs), ca.last_error()


@pytest.mark.parametrize("ops", [
    [("relu", 0, 0)],                 # its own value: would loop forever
    [("relu", 5, 0)],                 # a later op
    [("relu", -3, 0)],                # input 2 of 1
    [("relu", -1, 0), ("add", 0, 1)],  # the second operand names the op itself
    [("relu", -2147483648, 0)],       # INT_MIN: -(src + 1) must not overflow
])
def test_fused_chain_rejects_bad_operands(ops):
    rc, msg = _chain_status(ops)
    assert rc == -ca.ERR_INVALID
    assert "neither an earlier op nor an input" in msg


def test_fused_chain_checks_structure_before_handles():
    # a well-formed chain gets as far as the (NULL) input handle
    rc, msg = _chain_status([("relu", -1, 0), ("add", 0, -1)])
    assert rc == -ca.ERR_INVALID and "input is NULL" in msg
    rc, msg = _chain_status([("softmax", -1, 0)])
    assert rc == -ca.ERR_INVALID and "not elementwise" in msg


# ---------------------------------------------------------------------------
# planner: chain launch limits, RoPE and the FlashAttention pattern
# ---------------------------------------------------------------------------

def _step_io(model):
    """(name, ins, outs) per step from describe()."""
    out = []
    for line in model.describe().strip().splitlines()[:-1]:
        name = line.split(" ")[0]
        ins = line[line.index("in=(") + 4:line.index(")", line.index("in=("))]
        outs = line[line.index("out=(") + 5:line.rindex(")")]
        out.append((name, [int(x) for x in ins.split(",") if x],
                    [int(x) for x in outs.split(",") if x]))
    return out


def test_plan_splits_chains_at_sixteen_inputs():
    # a sum of 20 inputs: one chain would need 20 inputs, run_chain takes 16
    g = ca.Graph()
    xs = [g.input("64,64") for _ in range(20)]
    acc = xs[0]
    for x in xs[1:]:
        acc = g.op("add", acc, x)
    m = g.compile([acc])
    io = _step_io(m)
    assert len(io) == 2 and all(n.startswith("Fused") for n, _, _ in io)
    assert all(len(ins) <= 16 and len(outs) <= 16 for _, ins, outs in io)
    # the first chain's last value feeds the second chain
    assert io[0][2][-1] in io[1][1]


def test_plan_splits_chains_at_sixteen_stores():
    # a 20-op chain whose every value is requested: at most 16 stores per launch
    g = ca.Graph()
    x = g.input("128")
    vals, v = [], x
    for i in range(20):
        v = g.op("sin" if i % 2 else "cos", v)
        vals.append(v)
    m = g.compile(vals)
    io = _step_io(m)
    assert len(io) == 2
    assert all(len(outs) <= 16 for _, _, outs in io)
    stored = [o for _, _, outs in io for o in outs]
    assert sorted(stored) == sorted(vals)


def attention_graph(S=64, X=128, D=64, q_pos=3, k_pos=5, scale=True, sk=None):
    g = ca.Graph()
    q = g.input(f"{S},{X}")
    k = g.input(f"{sk or S},{X}")
    v = g.input(f"{sk or S},{X}")
    qr = g.rope(q, D, q_pos)
    kr = g.rope(k, D, k_pos)
    qs = g.op("scalar_mul", qr, param=1.0 / np.sqrt(D)) if scale else qr
    y = g.op("matmul", g.op("softmax", g.op("matmul", qs, kr)), v)
    return g, (q, k, v, qr, kr, qs), y


def test_plan_flash_attention_pattern():
    # lazy.rs:1621-1690: MatMul(Softmax(MatMul(ScalarMul(RoPE q), RoPE k)), v)
    # is one step reading the un-rotated q, k and v
    g, (q, k, v, *_), y = attention_graph()
    m = g.compile([y])
    io = _step_io(m)
    assert [n for n, _, _ in io] == ["FlashAttention(q_pos=3,k_pos=5,head_dim=64,causal)"]
    assert io[0][1] == [q, k, v] and io[0][2] == [y]
    # without the ScalarMul (the reference's kernel scales by 1/sqrt(D) anyway)
    g, (q, k, v, *_), y = attention_graph(scale=False)
    assert _step_io(g.compile([y]))[0][1] == [q, k, v]


def test_plan_flash_attention_non_matches():
    # no RoPE on k: planned op by op
    g = ca.Graph()
    q, k, v = g.input("64,128"), g.input("128,64"), g.input("64,128")
    y = g.op("matmul", g.op("softmax", g.op("matmul", g.rope(q, 64), k)), v)
    assert steps(g.compile([y])) == ["RoPE(0,64)", "MatMul+Softmax", "MatMul"]
    # every even head_dim up to 256 has an attention kernel (32, 80, 96 here)
    for D in (32, 80, 96):
        g, _, y = attention_graph(X=2 * D, D=D)
        assert f"FlashAttention(q_pos=3,k_pos=5,head_dim={D},causal)" in g.compile([y]).describe()
    # a hidden size that is not whole heads (RoPE zeroes the partial head)
    g, _, y = attention_graph(X=160, D=96)
    assert "FlashAttention" not in g.compile([y]).describe()
    # the scores are requested too: they must be materialised
    g, _, y = attention_graph()
    scores = y - 1
    assert "FlashAttention" not in g.compile([y, scores]).describe()
    # different head dims on q and k
    g = ca.Graph()
    q, k, v = g.input("64,128"), g.input("64,128"), g.input("64,128")
    y = g.op("matmul", g.op("softmax", g.op("matmul", g.rope(q, 64), g.rope(k, 128))), v)
    assert "FlashAttention" not in g.compile([y]).describe()


def test_plan_flash_attention_keeps_shared_nodes():
    # the rotated k is also an output: its RoPE keeps a step of its own, and
    # the fused step still reads the un-rotated k
    g, (q, k, v, qr, kr, qs), y = attention_graph()
    m = g.compile([y, kr])
    io = _step_io(m)
    names = [n for n, _, _ in io]
    assert names[0] == "RoPE(5,64)" and names[1].startswith("FlashAttention")
    assert io[1][1] == [q, k, v]


def test_plan_flash_attention_same_input_for_q_and_k():
    # self-attention on one tensor: q and k are the same node; its buffer is
    # released once (a duplicate release would hand one buffer to two values)
    g = ca.Graph()
    x, v = g.input("64,128"), g.input("64,128")
    y = g.op("matmul", g.op("softmax", g.op("matmul", g.rope(x, 64, 2), g.rope(x, 64, 2))), v)
    z = g.op("relu", y)
    m = g.compile([z])
    assert steps(m)[0].startswith("FlashAttention") and steps(m)[1] == "Fused[ReLU]"


def test_plan_matmul_of_a_node_with_itself():
    # MatMul(a, a) reads a twice: a's buffer is released once, so the two
    # values planned after it get different buffers
    g = ca.Graph()
    x = g.input("16,16")
    a = g.op("relu", x)
    p = g.op("matmul", a, a)
    s1 = g.op("sin", p)
    s2 = g.op("cos", p)
    y = g.op("matmul", s1, s2)
    m = g.compile([y])
    assert "vbufs=3" in m.describe(), m.describe()


def test_graph_rope_rejects_bad_parameters():
    g = ca.Graph()
    x = g.input("4,8")
    for hd in (0, 3, 258):
        with pytest.raises(ca.CloveError):
            g.rope(x, hd)
    with pytest.raises(ca.CloveError):
        g.rope(99, 8)
    with pytest.raises(ca.CloveError):
        g.op("rope", x)          # two integer parameters: only through graph_rope

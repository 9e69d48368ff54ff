// graph.cpp -- lazy tracing, planning and execution for the hot-path IR.
//
// The counterpart of Clove's LazyBackend tracer (lazy.rs:36-1153),
// compile() (lazy.rs:4273-5302) and CompiledModel::execute
// (lazy.rs:2545-4271), restricted to the opcodes of the hot path:
// Input, MatMul, the elementwise ops, Softmax, LayerNorm, PagedAttention.
//
// Passes, in the reference's order:
//   1. dead-code elimination from the requested outputs (lazy.rs:1553-1571);
//   2. constant folding of ScalarMul(1.0) (lazy.rs:1573-1598), skipping
//      nodes without an operand (the reference indexes dependencies[0] of
//      such nodes, e.g. the ones() seed of backward, and panics);
//   3. planning (lazy.rs:1610-2496): consecutive elementwise nodes with the
//      same element count form one fused chain; MatMul, Softmax, LayerNorm
//      and PagedAttention are barriers that flush the chain.  Every chain
//      value consumed outside its chain or requested as an output is stored
//      (the reference stores only the chain's last value, lazy.rs:1823).
//      A MatMul whose only consumer is Add(matmul, bias), optionally followed
//      by a ReLU or GELU that is the Add's only consumer, becomes one GEMM
//      step with the bias and activation applied in its store (the
//      Linear::forward pattern, nn.rs:115-118); the reference runs these as
//      separate passes;
//   4. liveness (lazy.rs:2500-2535): step outputs share virtual buffers
//      whose last reader has already run; buffers live in the model and grow
//      on demand (the reference reallocates at 2x, lazy.rs:2585-2607).
// Execution binds inputs in Input-node creation order (the reference binds
// by node id, which coincides for inputs traced first, lazy.rs:2618-2619),
// evaluates symbolic shapes with the S0..S3 environment, and returns fresh
// tensors for the requested outputs, so results never alias model buffers.
#include <algorithm>
#include <cctype>
#include <cmath>
#include <map>
#include <memory>
#include <set>
#include <sstream>

#include "common.hpp"
#include "graph.hpp"
#include "kernels/ew_abi.h"
#include "kernels/launch.hpp"
#include "runtime.hpp"

namespace clove {

// ---- SymInt ------------------------------------------------------------------

int64_t SymExpr::eval(const int64_t *env) const {
    switch (kind) {
    case CONST: return value;
    case SYM: return env ? env[value] : 1;  // backend.rs:43: unknown symbol -> 1
    case ADD: return a->eval(env) + b->eval(env);
    case SUB: {  // backend.rs:45: saturating_sub
        const int64_t x = a->eval(env), y = b->eval(env);
        return x > y ? x - y : 0;
    }
    default: return a->eval(env) * b->eval(env);
    }
}

std::string SymExpr::str() const {
    switch (kind) {
    case CONST: return std::to_string(value);
    case SYM: return "S" + std::to_string(value);
    case ADD: return "(" + a->str() + "+" + b->str() + ")";
    case SUB: return "(" + a->str() + "-" + b->str() + ")";
    default: return "(" + a->str() + "*" + b->str() + ")";
    }
}

SymPtr SymExpr::constant(int64_t v) {
    auto e = std::make_shared<SymExpr>();
    e->kind = CONST;
    e->value = v;
    return e;
}

SymPtr SymExpr::binop(int kind, SymPtr a, SymPtr b) {
    auto e = std::make_shared<SymExpr>();
    e->kind = kind;
    e->a = std::move(a);
    e->b = std::move(b);
    return e;
}

namespace {

struct Parser {
    const std::string &s;
    size_t i = 0;
    explicit Parser(const std::string &src) : s(src) {}
    void ws() {
        while (i < s.size() && std::isspace((unsigned char)s[i])) ++i;
    }
    [[noreturn]] void bad(const std::string &why) {
        fail(CLOVE_HIP_ERR_INVALID, "shape \"" + s + "\": " + why + " at offset " + std::to_string(i));
    }
    SymPtr factor() {
        ws();
        if (i < s.size() && s[i] == '(') {
            ++i;
            SymPtr e = expr();
            ws();
            if (i >= s.size() || s[i] != ')') bad("expected ')'");
            ++i;
            return e;
        }
        if (i < s.size() && s[i] == 'S') {
            ++i;
            if (i >= s.size() || s[i] < '0' || s[i] > '3') bad("symbols are S0..S3");
            auto e = std::make_shared<SymExpr>();
            e->kind = SymExpr::SYM;
            e->value = s[i++] - '0';
            return e;
        }
        if (i < s.size() && std::isdigit((unsigned char)s[i])) {
            int64_t v = 0;
            while (i < s.size() && std::isdigit((unsigned char)s[i])) v = v * 10 + (s[i++] - '0');
            return SymExpr::constant(v);
        }
        bad("expected a number, S0..S3 or '('");
    }
    SymPtr term() {
        SymPtr e = factor();
        for (;;) {
            ws();
            if (i < s.size() && s[i] == '*') {
                ++i;
                e = SymExpr::binop(SymExpr::MUL, e, factor());
            } else {
                return e;
            }
        }
    }
    SymPtr expr() {
        SymPtr e = term();
        for (;;) {
            ws();
            if (i < s.size() && (s[i] == '+' || s[i] == '-')) {
                const int k = s[i++] == '+' ? SymExpr::ADD : SymExpr::SUB;
                e = SymExpr::binop(k, e, term());
            } else {
                return e;
            }
        }
    }
};

SymPtr product(const std::vector<SymPtr> &shape) {
    if (shape.empty()) return SymExpr::constant(1);
    SymPtr e = shape[0];
    for (size_t i = 1; i < shape.size(); ++i) e = SymExpr::binop(SymExpr::MUL, e, shape[i]);
    return e;
}

std::string shape_key(const std::vector<SymPtr> &shape) { return product(shape)->str(); }

const char *op_name(int op) {
    switch (op) {
    case CLOVE_OP_INPUT: return "Input";
    case CLOVE_OP_MATMUL: return "MatMul";
    case CLOVE_OP_ADD: return "Add";
    case CLOVE_OP_SUB: return "Sub";
    case CLOVE_OP_MUL: return "Mul";
    case CLOVE_OP_SCALAR_MUL: return "ScalarMul";
    case CLOVE_OP_FLATTEN: return "Flatten";
    case CLOVE_OP_RELU: return "ReLU";
    case CLOVE_OP_GELU: return "GELU";
    case CLOVE_OP_SIN: return "Sin";
    case CLOVE_OP_COS: return "Cos";
    case CLOVE_OP_SOFTMAX: return "Softmax";
    case CLOVE_OP_LAYER_NORM: return "LayerNorm";
    case CLOVE_OP_DROPOUT: return "Dropout";
    case CLOVE_OP_RELU_GRAD: return "ReluGrad";
    case CLOVE_OP_GELU_GRAD: return "GeluGrad";
    case CLOVE_OP_CAST: return "Cast";
    case CLOVE_OP_SIGMOID: return "Sigmoid";
    case CLOVE_OP_TANH: return "Tanh";
    case CLOVE_OP_PAGED_ATTENTION: return "PagedAttention";
    case CLOVE_OP_ROPE: return "RoPE";
    default: return "?";
    }
}

}  // namespace

std::vector<SymPtr> parse_shape(const std::string &spec) {
    std::vector<SymPtr> dims;
    std::string cur;
    std::stringstream ss(spec);
    while (std::getline(ss, cur, ',')) {
        Parser p(cur);
        SymPtr e = p.expr();
        p.ws();
        if (p.i != cur.size()) p.bad("trailing characters");
        dims.push_back(e);
    }
    CLOVE_REQUIRE(!dims.empty(), CLOVE_HIP_ERR_INVALID, "empty shape");
    return dims;
}

// ---- tracing -----------------------------------------------------------------

int Graph::add_input(const std::string &spec) {
    Node n;
    n.id = (int)nodes.size();
    n.op = CLOVE_OP_INPUT;
    n.shape = parse_shape(spec);
    nodes.push_back(n);
    input_order.push_back(n.id);
    return n.id;
}

int Graph::add_op(int op, const std::vector<int> &deps, float param) {
    for (int d : deps)
        CLOVE_REQUIRE(d >= 0 && d < (int)nodes.size(), CLOVE_HIP_ERR_INVALID,
                      std::string(op_name(op)) + ": operand " + std::to_string(d) + " does not exist");
    Node n;
    n.id = (int)nodes.size();
    n.op = op;
    n.deps = deps;
    n.param = param;
    auto want = [&](size_t k) {
        CLOVE_REQUIRE(deps.size() == k, CLOVE_HIP_ERR_INVALID,
                      std::string(op_name(op)) + " takes " + std::to_string(k) + " operands");
    };
    const int ar = ew_arity(op);
    if (ar > 0) {
        want((size_t)ar);
        if (op == CLOVE_OP_FLATTEN)  // lazy.rs:571-580: [1, numel]
            n.shape = {SymExpr::constant(1), product(nodes[deps[0]].shape)};
        else
            n.shape = nodes[deps[0]].shape;  // lazy.rs:206: the first operand's shape
    } else if (op == CLOVE_OP_MATMUL) {   // lazy.rs:266-277
        want(2);
        const auto &bs = nodes[deps[1]].shape;
        CLOVE_REQUIRE(bs.size() == 2, CLOVE_HIP_ERR_SHAPE, "MatMul: b must be 2-d");
        n.shape = nodes[deps[0]].shape;
        n.shape.back() = bs[1];
    } else if (op == CLOVE_OP_SOFTMAX) {
        want(1);
        n.shape = nodes[deps[0]].shape;
    } else if (op == CLOVE_OP_LAYER_NORM) {
        want(3);
        n.shape = nodes[deps[0]].shape;
    } else if (op == CLOVE_OP_PAGED_ATTENTION) {  // lazy.rs:860-886: q's shape
        want(6);
        n.shape = nodes[deps[0]].shape;
    } else if (op == CLOVE_OP_ROPE) {
        fail(CLOVE_HIP_ERR_INVALID, "RoPE takes two integer parameters: use clove_hip_graph_rope");
    } else {
        fail(CLOVE_HIP_ERR_INVALID, "opcode " + std::to_string(op) + " is not on the hot path");
    }
    nodes.push_back(n);
    return n.id;
}

// lazy.rs:475-480: RoPE(pos_offset, head_dim) keeps its operand's shape.
int Graph::add_rope(int x, int64_t pos_offset, int64_t head_dim) {
    CLOVE_REQUIRE(x >= 0 && x < (int)nodes.size(), CLOVE_HIP_ERR_INVALID,
                  "RoPE: operand " + std::to_string(x) + " does not exist");
    CLOVE_REQUIRE(head_dim >= 2 && head_dim % 2 == 0 && head_dim <= 256, CLOVE_HIP_ERR_SHAPE,
                  "RoPE: head_dim must be even and at most 256");
    CLOVE_REQUIRE(pos_offset >= 0 && pos_offset < (1 << 30), CLOVE_HIP_ERR_INVALID,
                  "RoPE: pos_offset must be in [0, 2^30)");
    Node n;
    n.id = (int)nodes.size();
    n.op = CLOVE_OP_ROPE;
    n.deps = {x};
    n.shape = nodes[x].shape;
    n.pos_offset = pos_offset;
    n.head_dim = head_dim;
    nodes.push_back(n);
    return n.id;
}

// ---- compile -----------------------------------------------------------------

Model::Model(const Graph &g, const std::vector<int> &outs) : nodes(g.nodes), inputs(g.input_order), outputs(outs) {
    for (int o : outs)
        CLOVE_REQUIRE(o >= 0 && o < (int)nodes.size(), CLOVE_HIP_ERR_INVALID,
                      "output node " + std::to_string(o) + " does not exist");
    CLOVE_REQUIRE(!outs.empty(), CLOVE_HIP_ERR_INVALID, "no outputs requested");

    // 1. dead-code elimination
    std::vector<char> alive(nodes.size(), 0);
    std::vector<int> stack(outs.begin(), outs.end());
    while (!stack.empty()) {
        const int id = stack.back();
        stack.pop_back();
        if (alive[id]) continue;
        alive[id] = 1;
        for (int d : nodes[id].deps) stack.push_back(d);
    }
    // 2. constant folding: x * 1.0 is x.  A folded node that is itself an
    // output stays (it must produce a buffer).
    std::vector<int> alias(nodes.size());
    for (size_t i = 0; i < nodes.size(); ++i) alias[i] = (int)i;
    std::set<int> out_set(outs.begin(), outs.end());
    // Nodes whose first operand was a folded x * 1.0: the attention pattern
    // below reads that as a softmax scale of 1.
    std::set<int> unit_scaled_lhs;
    for (auto &n : nodes) {
        if (!alive[n.id]) continue;
        if (!n.deps.empty() && alias[n.deps[0]] != n.deps[0]) unit_scaled_lhs.insert(n.id);
        for (int &d : n.deps) d = alias[d];
        if (n.op == CLOVE_OP_SCALAR_MUL && !n.deps.empty() &&
            std::fabs(n.param - 1.0f) < 1.1920929e-7f && !out_set.count(n.id)) {
            alias[n.id] = n.deps[0];
            alive[n.id] = 0;
            ++folded;
        }
    }
    for (const Node &n : nodes)
        if (alive[n.id]) ++live_nodes;

    // Consumers of each node, for deciding what a chain must store.
    std::vector<std::vector<int>> users(nodes.size());
    for (const Node &n : nodes)
        if (alive[n.id])
            for (int d : n.deps) users[d].push_back(n.id);

    // `sole(id)`: the only consumer of `id`, or -1 when it has several, none,
    // or is a requested output.
    auto sole = [&](int id) {
        return (!out_set.count(id) && users[id].size() == 1) ? users[id][0] : -1;
    };
    std::set<int> absorbed;  // nodes folded into another step

    // 2b. The FlashAttention pattern (lazy.rs:1621-1690):
    //   MatMul(Softmax(MatMul([ScalarMul(s)](RoPE(q)), RoPE(k))), v)
    // becomes one ATTENTION step over the un-rotated q and k and v, with the
    // contract of the reference's fused kernel (lazy.rs:4821-4909): one token
    // per row, keys after the query's row masked, q and k rotated at the
    // RoPE nodes' positions, head_dim from the RoPE nodes (here heads =
    // hidden / head_dim; the reference kernel takes one head).  The softmax
    // scale is the ScalarMul's factor (a folded x * 1.0 counts as a factor of
    // 1), 1/sqrt(head_dim) without one (the
    // reference kernel always uses 1/sqrt(head_dim) and drops the
    // ScalarMul, which is the same thing in MultiHeadAttention::forward,
    // nn/attention.rs:62-67).  Both RoPE nodes must be present with one
    // head_dim the kernel supports, q must be 2-d, and the inner MatMul and
    // the Softmax must feed only the pattern; otherwise the nodes are planned
    // one by one.  A RoPE or ScalarMul node that other nodes also read keeps
    // its own step; the fused step still starts from the un-rotated inputs.
    std::map<int, Step> attention_at;  // outer MatMul id -> its ATTENTION step
    for (const Node &outer : nodes) {
        if (!alive[outer.id] || outer.op != CLOVE_OP_MATMUL) continue;
        const int sm = outer.deps[0], v = outer.deps[1];
        if (nodes[sm].op != CLOVE_OP_SOFTMAX || sole(sm) != outer.id) continue;
        const int inner = nodes[sm].deps[0];
        if (nodes[inner].op != CLOVE_OP_MATMUL || sole(inner) != sm) continue;
        int qq = nodes[inner].deps[0];
        const int kk = nodes[inner].deps[1];
        float scale = unit_scaled_lhs.count(inner) ? 1.0f : 0.0f;
        int smul = -1;
        if (nodes[qq].op == CLOVE_OP_SCALAR_MUL) {
            scale = nodes[qq].param;
            smul = qq;
            qq = nodes[qq].deps[0];
        }
        if (nodes[qq].op != CLOVE_OP_ROPE || nodes[kk].op != CLOVE_OP_ROPE || qq == kk) continue;
        const int64_t hd = nodes[qq].head_dim;
        if (nodes[kk].head_dim != hd || !k::attention_supported((int)hd)) continue;
        const int q = nodes[qq].deps[0], kx = nodes[kk].deps[0];
        if (nodes[q].shape.size() != 2 || nodes[kx].shape.size() != 2 ||
            nodes[v].shape.size() != 2)
            continue;
        // whole heads only: a RoPE over a hidden size with a partial last head
        // zeroes that head's dims, which the fused step would not reproduce
        auto whole_heads = [&](int id) {
            const SymExpr &x = *nodes[id].shape[1];
            return x.kind == SymExpr::CONST && x.value > 0 && x.value % hd == 0;
        };
        if (!whole_heads(q) || !whole_heads(kx) || !whole_heads(v)) continue;
        if (smul >= 0 && !(scale > 0.f)) continue;  // the kernel needs a positive scale
        Step st;
        st.kind = Step::ATTENTION;
        st.in = {q, kx, v};
        st.out = {outer.id};
        st.q_pos = nodes[qq].pos_offset;
        st.k_pos = nodes[kk].pos_offset;
        st.head_dim = hd;
        st.scale = scale;
        attention_at[outer.id] = st;
        absorbed.insert(sm);
        absorbed.insert(inner);
        const int after_q = smul >= 0 ? smul : inner;
        if (smul >= 0 && sole(smul) == inner) absorbed.insert(smul);
        if (sole(qq) == after_q) absorbed.insert(qq);
        if (sole(kk) == inner) absorbed.insert(kk);
    }

    // 3. planning
    std::vector<int> group;
    auto flush = [&]() {
        if (group.empty()) return;
        Step st;
        st.kind = Step::FUSED;
        std::set<int> members(group.begin(), group.end());
        std::map<int, int> pos;  // node id -> index in chain
        for (size_t i = 0; i < group.size(); ++i) pos[group[i]] = (int)i;
        for (size_t i = 0; i < group.size(); ++i) {
            const Node &n = nodes[group[i]];
            ChainOp op;
            op.opcode = n.op;
            op.param = n.param;
            int srcs[2] = {0, 0};
            for (size_t j = 0; j < n.deps.size(); ++j) {
                const int d = n.deps[j];
                if (members.count(d)) {
                    srcs[j] = pos[d];
                } else {
                    auto it = std::find(st.in.begin(), st.in.end(), d);
                    int k = (int)(it - st.in.begin());
                    if (it == st.in.end()) st.in.push_back(d);
                    srcs[j] = -(k + 1);
                }
            }
            op.src0 = srcs[0];
            op.src1 = srcs[1];
            bool escapes = out_set.count(n.id) > 0;
            for (int u : users[n.id])
                if (!members.count(u)) escapes = true;
            op.store = escapes || i + 1 == group.size();
            if (op.store) st.out.push_back(n.id);
            st.chain.push_back(op);
        }
        st.numel = product(nodes[group.back()].shape);
        steps.push_back(st);
        group.clear();
    };
    // Whether `group` plus node `id` stays within what one chain launch
    // takes (run_chain: CL_MAX_IN distinct outside inputs, CL_MAX_OUT stored
    // values).  A member is stored when it is requested or read outside the
    // group, and the last member always is, exactly as flush() decides.
    auto fits_with = [&](int id) {
        std::set<int> members(group.begin(), group.end());
        members.insert(id);
        std::set<int> outside;
        int stores = 0;
        for (int m : members) {
            for (int d : nodes[m].deps)
                if (!members.count(d)) outside.insert(d);
            bool escapes = out_set.count(m) > 0 || m == id;
            for (int u : users[m])
                if (!members.count(u)) escapes = true;
            stores += escapes;
        }
        return (int)outside.size() <= CL_MAX_IN && stores <= CL_MAX_OUT;
    };
    for (const Node &n : nodes) {
        if (!alive[n.id] || n.op == CLOVE_OP_INPUT || absorbed.count(n.id)) continue;
        if (attention_at.count(n.id)) {
            flush();
            steps.push_back(attention_at[n.id]);
            continue;
        }
        if (ew_arity(n.op) > 0) {
            if (!group.empty() &&
                (shape_key(nodes[group.back()].shape) != shape_key(n.shape) ||
                 (int)group.size() >= 32 || !fits_with(n.id)))
                flush();
            group.push_back(n.id);
            continue;
        }
        flush();
        Step st;
        switch (n.op) {
        case CLOVE_OP_MATMUL: st.kind = Step::MATMUL; break;
        case CLOVE_OP_SOFTMAX: st.kind = Step::SOFTMAX; break;
        case CLOVE_OP_LAYER_NORM: st.kind = Step::LAYER_NORM; break;
        case CLOVE_OP_ROPE:
            st.kind = Step::ROPE;
            st.q_pos = n.pos_offset;
            st.head_dim = n.head_dim;
            break;
        default: st.kind = Step::PAGED; break;
        }
        st.in = n.deps;
        st.out = {n.id};
        if (n.op == CLOVE_OP_MATMUL) {
            // Epilogue fusion.
            int tail = n.id;
            const int add = sole(n.id);
            if (add >= 0 && nodes[add].op == CLOVE_OP_ADD && nodes[add].deps[0] == n.id &&
                nodes[add].deps[1] != n.id) {
                const int bias = nodes[add].deps[1];
                // the bias must already exist when this step runs
                if (nodes[bias].op == CLOVE_OP_INPUT || bias < n.id) {
                    st.in.push_back(bias);
                    absorbed.insert(add);
                    tail = add;
                }
            }
            const int act = sole(tail);
            if (act >= 0 && nodes[act].deps[0] == tail &&
                (nodes[act].op == CLOVE_OP_RELU || nodes[act].op == CLOVE_OP_GELU)) {
                st.act = nodes[act].op == CLOVE_OP_RELU ? 1 : 2;
                absorbed.insert(act);
                tail = act;
            } else if (act >= 0 && nodes[act].op == CLOVE_OP_SOFTMAX && nodes[act].deps[0] == tail) {
                // a classifier head (MatMul [-> Add] -> Softmax, rows over the
                // last dim): one step; the GEMM applies the softmax itself
                // when a tile holds whole rows, else it runs after the GEMM
                st.act = 3;
                absorbed.insert(act);
                tail = act;
            }
            st.out = {tail};
        }
        steps.push_back(st);
    }
    flush();

    // 3b. Horizontal MatMul groups (lazy.rs:2443-2493): a run of consecutive
    // MatMul steps none of which reads another's output becomes one step that
    // runs as one grouped launch.  (The reference only checks each candidate
    // against the first member's output; every earlier member is checked
    // here.)
    {
        std::vector<Step> grouped;
        for (size_t i = 0; i < steps.size();) {
            if (steps[i].kind != Step::MATMUL) {
                grouped.push_back(steps[i++]);
                continue;
            }
            std::vector<Step> run{steps[i]};
            std::set<int> written(steps[i].out.begin(), steps[i].out.end());
            size_t j = i + 1;
            for (; j < steps.size() && steps[j].kind == Step::MATMUL; ++j) {
                bool reads_member = false;
                for (int d : steps[j].in) reads_member = reads_member || written.count(d) > 0;
                if (reads_member) break;
                run.push_back(steps[j]);
                written.insert(steps[j].out.begin(), steps[j].out.end());
            }
            if (run.size() == 1) {
                grouped.push_back(run[0]);
            } else {
                Step g;
                g.kind = Step::MATMUL_GROUP;
                std::set<int> seen;
                for (const Step &m : run) {
                    for (int d : m.in)
                        if (seen.insert(d).second) g.in.push_back(d);
                    g.out.insert(g.out.end(), m.out.begin(), m.out.end());
                }
                g.members = run;
                grouped.push_back(g);
            }
            i = j;
        }
        steps.swap(grouped);
    }

    // 4. liveness: a virtual buffer is released after the last step reading it.
    std::map<int, int> last_use;
    for (size_t i = 0; i < steps.size(); ++i)
        for (int d : steps[i].in) last_use[d] = (int)i;
    std::vector<int> free_list;
    for (size_t i = 0; i < steps.size(); ++i) {
        for (int o : steps[i].out) {
            if (!free_list.empty()) {
                vbuf[o] = free_list.back();
                free_list.pop_back();
            } else {
                vbuf[o] = num_vbufs++;
            }
        }
        // each buffer is released once, however many operands of the step
        // read it (MatMul(a, a), attention with q and k from one node)
        std::set<int> read(steps[i].in.begin(), steps[i].in.end());
        for (int d : read) {
            auto it = vbuf.find(d);
            if (it != vbuf.end() && last_use[d] == (int)i && !out_set.count(d))
                free_list.push_back(it->second);
        }
    }
}

static std::string matmul_name(const Step &st) {
    return std::string("MatMul") + (st.in.size() > 2 ? "+Add" : "") +
           (st.act == 1 ? "+ReLU" : st.act == 2 ? "+GELU" : st.act == 3 ? "+Softmax" : "");
}

std::string Model::describe() const {
    std::ostringstream s;
    for (const Step &st : steps) {
        switch (st.kind) {
        case Step::FUSED: {
            s << "Fused[";
            for (size_t i = 0; i < st.chain.size(); ++i)
                s << (i ? "," : "") << op_name(st.chain[i].opcode);
            s << "]";
            break;
        }
        case Step::MATMUL: s << matmul_name(st); break;
        case Step::MATMUL_GROUP:
            s << "MatMulGroup[";
            for (size_t i = 0; i < st.members.size(); ++i)
                s << (i ? "," : "") << matmul_name(st.members[i]);
            s << "]";
            break;
        case Step::SOFTMAX: s << "Softmax"; break;
        case Step::LAYER_NORM: s << "LayerNorm"; break;
        case Step::ROPE: s << "RoPE(" << st.q_pos << "," << st.head_dim << ")"; break;
        case Step::ATTENTION:
            s << "FlashAttention(q_pos=" << st.q_pos << ",k_pos=" << st.k_pos
              << ",head_dim=" << st.head_dim << ",causal)";
            break;
        default: s << "PagedAttention"; break;
        }
        s << " in=(";
        for (size_t i = 0; i < st.in.size(); ++i) s << (i ? "," : "") << st.in[i];
        s << ") out=(";
        for (size_t i = 0; i < st.out.size(); ++i) s << (i ? "," : "") << st.out[i];
        s << ")\n";
    }
    s << "vbufs=" << num_vbufs << " folded=" << folded << " live=" << live_nodes << "\n";
    return s.str();
}

// ---- execute -----------------------------------------------------------------

std::vector<TensorNode> Model::execute(const std::vector<TensorNode> &in, const int64_t *env) {
    CLOVE_REQUIRE(in.size() == inputs.size(), CLOVE_HIP_ERR_INVALID,
                  "model has " + std::to_string(inputs.size()) + " inputs, got " +
                      std::to_string(in.size()));
    std::map<int, const Tensor *> bound;
    for (size_t i = 0; i < inputs.size(); ++i) {
        CLOVE_REQUIRE(in[i] != nullptr, CLOVE_HIP_ERR_INVALID, "input " + std::to_string(i) + " is NULL");
        const Node &n = nodes[inputs[i]];
        const int64_t want = product(n.shape)->eval(env);
        CLOVE_REQUIRE((int64_t)in[i]->numel == want, CLOVE_HIP_ERR_SHAPE,
                      "input " + std::to_string(i) + " has " + std::to_string(in[i]->numel) +
                          " elements, the graph expects " + std::to_string(want));
        bound[inputs[i]] = in[i].get();
    }

    // Evaluate shapes and size the virtual buffers.
    auto eval_shape = [&](int id) {
        std::vector<size_t> s;
        for (const SymPtr &d : nodes[id].shape) s.push_back((size_t)std::max<int64_t>(0, d->eval(env)));
        return s;
    };
    std::vector<size_t> need(num_vbufs, 0);
    for (const auto &kv : vbuf) need[kv.second] = std::max(need[kv.second], numel_of(eval_shape(kv.first)));
    if (buffers.size() < (size_t)num_vbufs) buffers.resize(num_vbufs);
    for (int v = 0; v < num_vbufs; ++v) {
        if (!buffers[v] || buffers[v]->numel < need[v]) {
            const size_t cap = need[v] < 256 ? 256 : need[v] * 2;
            buffers[v] = new_tensor({cap}, CLOVE_HIP_F32);
        }
    }
    // Views of the virtual buffers with each node's shape.
    std::map<int, std::unique_ptr<Tensor>> views;
    auto view_of = [&](int id) -> Tensor * {
        auto it = views.find(id);
        if (it != views.end()) return it->second.get();
        auto t = std::make_unique<Tensor>();
        t->owned = false;
        t->dtype = CLOVE_HIP_F32;
        t->shape = eval_shape(id);
        t->numel = numel_of(t->shape);
        const Tensor &buf = *buffers[vbuf.at(id)];
        t->data = buf.data;
        t->bytes = buf.bytes;
        Tensor *raw = t.get();
        views[id] = std::move(t);
        return raw;
    };
    auto arg = [&](int id) -> const Tensor * {
        auto it = bound.find(id);
        if (it != bound.end()) return it->second;
        return view_of(id);
    };
    // Outputs are fresh tensors, never aliases of model buffers or of each
    // other.  An output that a step computes is written by that step straight
    // into its fresh tensor (later steps read it from there), so no copy is
    // needed; an output that is a graph input, or a node listed twice, is
    // copied at the end.
    std::vector<TensorNode> result(outputs.size());
    for (size_t i = 0; i < outputs.size(); ++i) {
        const int o = outputs[i];
        if (bound.count(o) || views.count(o)) continue;
        TensorNode t = new_tensor(eval_shape(o), CLOVE_HIP_F32);
        auto v = std::make_unique<Tensor>();
        v->owned = false;
        v->dtype = CLOVE_HIP_F32;
        v->shape = t->shape;
        v->numel = t->numel;
        v->data = t->data;
        v->bytes = t->bytes;
        views[o] = std::move(v);
        result[i] = t;
    }

    for (const Step &st : steps) {
        switch (st.kind) {
        case Step::FUSED: {
            std::vector<const Tensor *> ins;
            for (int d : st.in) ins.push_back(arg(d));
            std::vector<Tensor *> outs;
            for (int o : st.out) outs.push_back(view_of(o));
            const int64_t n = st.numel->eval(env);
            run_chain(st.chain, ins, outs, (size_t)std::max<int64_t>(0, n));
            break;
        }
        case Step::MATMUL:
            HipBackend::matmul_into(*arg(st.in[0]), *arg(st.in[1]), *view_of(st.out[0]),
                                    st.in.size() > 2 ? arg(st.in[2]) : nullptr, st.act);
            break;
        case Step::MATMUL_GROUP: {
            std::vector<HipBackend::GemmMember> ms;
            for (const Step &m : st.members)
                ms.push_back({arg(m.in[0]), arg(m.in[1]), view_of(m.out[0]),
                              m.in.size() > 2 ? arg(m.in[2]) : nullptr, m.act});
            HipBackend::matmul_group_into(ms);
            break;
        }
        case Step::SOFTMAX:
            HipBackend::softmax_into(*arg(st.in[0]), *view_of(st.out[0]));
            break;
        case Step::LAYER_NORM:
            HipBackend::layer_norm_into(*arg(st.in[0]), *arg(st.in[1]), *arg(st.in[2]),
                                        *view_of(st.out[0]));
            break;
        case Step::ROPE:
            HipBackend::rope_into(*arg(st.in[0]), (size_t)st.q_pos, (size_t)st.head_dim,
                                  *view_of(st.out[0]));
            break;
        case Step::ATTENTION: {
            const Tensor *q = arg(st.in[0]);
            const int heads = (int)(q->shape.back() / (size_t)st.head_dim);
            CLOVE_REQUIRE(heads >= 1 && q->shape.back() % (size_t)st.head_dim == 0,
                          CLOVE_HIP_ERR_SHAPE,
                          "attention: the hidden size " + std::to_string(q->shape.back()) +
                              " is not a multiple of head_dim " + std::to_string(st.head_dim));
            HipBackend::flash_attention_into(*q, *arg(st.in[1]), *arg(st.in[2]), heads,
                                             (int)st.q_pos, (int)st.k_pos, 0, 0,
                                             CLOVE_ATTN_CAUSAL | CLOVE_ATTN_ROPE, st.scale,
                                             *view_of(st.out[0]));
            break;
        }
        case Step::PAGED: {
            const Tensor *q = arg(st.in[0]);
            const int D = (int)arg(st.in[3])->shape.back();
            HipBackend::paged_attention_into(*q, arg(st.in[1]), arg(st.in[2]), *arg(st.in[3]),
                                             *arg(st.in[4]), *arg(st.in[5]),
                                             1.0f / std::sqrt((float)D), *view_of(st.out[0]));
            break;
        }
        }
    }

    // The outputs not written in place: device-to-device copies on the stream.
    for (size_t i = 0; i < outputs.size(); ++i) {
        if (result[i]) continue;
        const Tensor *src = arg(outputs[i]);
        TensorNode t = new_tensor(src->shape, src->dtype);
        if (src->numel)
            CLOVE_HIP_CHECK(hipMemcpyAsync(t->data, src->data, src->numel * 4,
                                           hipMemcpyDeviceToDevice, ctx().stream));
        result[i] = t;
    }
    return result;
}

}  // namespace clove
